// gfx950 kernels of the fused token-sampling path.
//
// Per row the work is the reference's serving/sampling.py:44-63 (penalties, greedy or
// temperature -> top-k -> top-p -> draw, log-softmax, top-N), restructured for one
// streaming pass over the [B, V] logits:
//
//   scan_kernel     grid = B * S workgroups of 256 threads; workgroup (row, chunk)
//                   loads its chunk of E elements per thread into registers with
//                   16-byte loads, applies the penalties from an LDS count table of
//                   the row's history (owners of history elements penalise them in
//                   an LDS staging area), reduces max / argmax / sum-exp with wave64
//                   shuffles, and writes the chunk's candidates: every element at or
//                   above a lower bound on the chunk's K-th largest value, found by
//                   per-wave ballot bisections over the keys of register-group maxima.
//   row_kernel      one workgroup per row.  combine_row gathers the row's candidates
//                   (flattened over chunks) into LDS, narrows them with histogram and
//                   radix selects, rank-sorts the survivors, applies top-k / top-p
//                   exactly on them, draws by inverse CDF in vocab order, and writes
//                   token, logprob and top-N.  Rows the candidates cannot settle
//                   (top-p mass beyond the candidates, slot overflow on massive ties)
//                   take dense_resolve: radix selects over the whole row (count- and
//                   mass-weighted, 8-bit digits, LDS histograms).
//   probs_kernel    optional: the final probability vector of each row.
//
// The two main launches are separate kernels on purpose: handing a row to the last
// chunk workgroup would need a device-scope release per workgroup, which on gfx950 is
// an L2 writeback plus invalidate and costs more than the second launch.
//
// There is no dense contraction anywhere, so no MFMA: the streaming pass is bound by
// HBM bandwidth (bytes per row = V * sizeof(logit) + 4 * H).

#include <hip/hip_runtime.h>
#include <math.h>
#include <stdint.h>

#include <mutex>
#include <type_traits>

#include "internal.h"

namespace kls {
namespace {

constexpr float kNegInf = -__builtin_huge_valf();
constexpr double kFixScale = 1099511627776.0;  // 2^40: fixed-point unit of the row path's masses

__device__ __forceinline__ int lane_id() { return threadIdx.x & 63; }
__device__ __forceinline__ int wave_id() { return threadIdx.x >> 6; }

// Order-preserving 32-bit key of a float; -0.0 and +0.0 share a key because the
// reference's comparisons treat them as equal.
__device__ __forceinline__ uint32_t fkey(float y) {
    uint32_t u = __float_as_uint(y);
    if (u == 0x80000000u) u = 0u;
    return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}
__device__ __forceinline__ float fkey_inv(uint32_t k) {
    return __uint_as_float((k & 0x80000000u) ? (k & 0x7fffffffu) : ~k);
}

// exp(d) for d <= 0 via the hardware base-2 exponential; used for sums whose
// relative accuracy only needs to be ~1e-7.
__device__ __forceinline__ float exp_fast(float d) {
    return __builtin_amdgcn_exp2f(d * 1.4426950408889634f);
}

// Fixed-point weight (unit 2^-40) of a final score y under the row max m: integer sums
// are exact and independent of their order.  w * 2^40 (w = exp(y - m) <= 1) is exact in
// fp32, rounded half-to-even to an integer there, and split into two 32-bit halves, each
// converted exactly: the value of round((double)w * 2^40), in full-rate fp32 operations.
template <int kBits = 40>
__device__ __forceinline__ unsigned long long weight_fix(float y, float m) {
    const float f = __builtin_rintf(exp_fast(y - m) * (float)(1ull << kBits));
    const float h = __builtin_truncf(f * 2.3283064365386963e-10f);   // f / 2^32
    const float lo = __builtin_fmaf(h, -4294967296.0f, f);            // f - h * 2^32, exact
    return ((unsigned long long)(uint32_t)h << 32) | (uint32_t)lo;
}

__device__ __forceinline__ int row_mode(const klsample_row_params &p, int V) {
    if (p.flags & KLSAMPLE_ROW_GREEDY) return kGreedy;
    if (p.top_k > 0 && p.top_k < V) return kTopK;
    if (p.flags & KLSAMPLE_ROW_TOP_P) return kTopP;
    return kFull;
}

// Repetition penalty (serving/sampling.py:49: s*r if s<0 else s/r, fp32, true
// division), then presence/frequency: s - fp32(fp32(beta*count) + alpha), no FMA.
__device__ __forceinline__ float penalize(float s, uint32_t count, const klsample_row_params &p) {
    if (p.flags & KLSAMPLE_ROW_REPETITION)
        s = (s < 0.f) ? __fmul_rn(s, p.repetition_penalty) : __fdiv_rn(s, p.repetition_penalty);
    if (p.flags & KLSAMPLE_ROW_PRESENCE_FREQUENCY) {
        float t = __fmul_rn(p.frequency_penalty, (float)count);
        t = __fadd_rn(t, p.presence_penalty);
        s = __fsub_rn(s, t);
    }
    return s;
}

// The row's history as [h0, h1) in hist_ids: CSR offsets, or begin/end pairs
// (KLSAMPLE_OPT_HISTORY_PAIRS), in memory or (kInline) possibly in the kernel
// arguments.  Both 0 without history.
template <bool kInline = true>
__device__ __forceinline__ void hist_range(const Args &a, int row, int &h0, int &h1) {
    h0 = h1 = 0;
    const int i = (a.options & KLSAMPLE_OPT_HISTORY_PAIRS) ? 2 * row : row;
    if (kInline && (a.inline_flags & kInlineOffsets)) {
        h0 = a.inl_off[i];
        h1 = a.inl_off[i + 1];
        return;
    }
    if (a.hist_off == nullptr) return;
    h0 = a.hist_off[i];
    h1 = a.hist_off[i + 1];
}

// The row's parameters, from memory or from the kernel arguments.
__device__ __forceinline__ klsample_row_params row_params(const Args &a, int row) {
    return (a.inline_flags & kInlineParams) ? a.inl_params[row] : a.params[row];
}

__device__ __forceinline__ bool has_penalty(const Args &a, const klsample_row_params &p, int row) {
    if (!(p.flags & (KLSAMPLE_ROW_REPETITION | KLSAMPLE_ROW_PRESENCE_FREQUENCY))) return false;
    int h0, h1;
    hist_range(a, row, h0, h1);
    return h1 > h0;
}

// ---------------------------------------------------------------------------------
// LDS scratch shared by all phases of a workgroup.  Red is the cross-wave exchange
// slot of the block reductions.
struct Red {
    union {
        float f[kWaves];
        double d[kWaves];
        int i[kWaves];
        uint32_t u[kWaves];
        unsigned long long q[kWaves];
    } red;
};

// The streaming pass needs little beyond the reductions (its LDS footprint sets how
// many workgroups share a CU).
struct ScanMisc : Red {
    uint32_t wbound[kWaves];
    uint32_t bound_key;
    int ncand;
    // per-wave max, sum of exp relative to it, finite count and lowest argmax
    float wm[kWaves];
    double wz[kWaves];
    int wn[kWaves], wa[kWaves];
};

constexpr int kSegCap = 128;   // segments of an ordered search

struct TopPCut {
    float cut;
    int cut_idx;             // 0x7fffffff: every entry scoring cut is kept
    int kept;
    unsigned long long zf;   // kept mass (fixed point)
};

struct Misc : Red {
    float rf[2][kWaves];
    int ri[2][kWaves];
    uint32_t hist[256];
    uint32_t part[kThreads];   // block_rank_sort: per-thread partial ranks
    uint32_t irank[64];        // block_index_rank: vocab-order ranks of a kept list
    unsigned long long hmass[256];
    unsigned long long sink[kThreads];   // per-thread target of masked LDS stores
    int topn_idx[kMaxLogprobs];
    float topn_y[kMaxLogprobs];
    uint32_t bound_key;
    int ncand;
    int last;
    int flag;
    uint32_t sel_digit;
    uint32_t sel_need;
    unsigned long long sel_above_mass;
    uint32_t sel_above_count;
    int sel_found;
    int ia, ib;
    int ne;          // entries of a row's top set (top-k finish)
    uint32_t kmin, kmax;
    double da, db;
    TopPCut topp;
    double seg[kSegCap];    // ordered_find: per-segment weight sums
    int segl[kSegCap];      // ... and last positive item per segment
};

// ---------------------------------------------------------------------------------
// Wave64 primitives on DPP (no LDS round trip): quad_perm / row mirrors / row_bcast
// reduce a wave in six steps; row_shr + row_bcast give an inclusive scan and
// wave_shr:1 turns it exclusive.  Values wider than 32 bits move as two halves.
template <typename To, typename From>
__device__ __forceinline__ To bitcast(From v) { return __builtin_bit_cast(To, v); }

template <int CTRL, int ROW_MASK = 0xf, int BANK_MASK = 0xf>
__device__ __forceinline__ uint32_t dpp32(uint32_t old, uint32_t v) {
    return (uint32_t)__builtin_amdgcn_update_dpp((int)old, (int)v, CTRL, ROW_MASK, BANK_MASK, false);
}

template <int CTRL, int ROW_MASK = 0xf, int BANK_MASK = 0xf, typename T>
__device__ __forceinline__ T dpp(T old, T v) {
    if constexpr (sizeof(T) == 4) {
        return bitcast<T>(dpp32<CTRL, ROW_MASK, BANK_MASK>(bitcast<uint32_t>(old), bitcast<uint32_t>(v)));
    } else {
        const uint64_t o = bitcast<uint64_t>(old), x = bitcast<uint64_t>(v);
        const uint32_t lo = dpp32<CTRL, ROW_MASK, BANK_MASK>((uint32_t)o, (uint32_t)x);
        const uint32_t hi = dpp32<CTRL, ROW_MASK, BANK_MASK>((uint32_t)(o >> 32), (uint32_t)(x >> 32));
        return bitcast<T>(((uint64_t)hi << 32) | lo);
    }
}

template <typename T>
__device__ __forceinline__ T readlane(T v, int lane) {
    if constexpr (sizeof(T) == 4) {
        return bitcast<T>((uint32_t)__builtin_amdgcn_readlane((int)bitcast<uint32_t>(v), lane));
    } else {
        const uint64_t x = bitcast<uint64_t>(v);
        const uint32_t lo = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)x, lane);
        const uint32_t hi = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)(x >> 32), lane);
        return bitcast<T>(((uint64_t)hi << 32) | lo);
    }
}

// Reduction over the 64 lanes of a fully active wave; the result is wave-uniform.
template <typename T, typename Op>
__device__ __forceinline__ T wave_reduce(T v, Op op, T id) {
    v = op(v, dpp<0xb1>(id, v));         // quad_perm [1,0,3,2]
    v = op(v, dpp<0x4e>(id, v));         // quad_perm [2,3,0,1]
    v = op(v, dpp<0x141>(id, v));        // row_half_mirror
    v = op(v, dpp<0x140>(id, v));        // row_mirror
    v = op(v, dpp<0x142, 0xa>(id, v));   // row_bcast:15 into rows 1 and 3
    v = op(v, dpp<0x143, 0xc>(id, v));   // row_bcast:31 into rows 2 and 3
    return readlane(v, 63);
}

// Inclusive prefix sum over the lanes of a fully active wave.
template <typename T>
__device__ __forceinline__ T wave_incl_scan(T v) {
    const T z = T(0);
    v = v + dpp<0x111>(z, v);            // row_shr:1
    v = v + dpp<0x112>(z, v);            // row_shr:2
    v = v + dpp<0x114>(z, v);            // row_shr:4
    v = v + dpp<0x118>(z, v);            // row_shr:8
    v = v + dpp<0x142, 0xa>(z, v);       // row_bcast:15
    v = v + dpp<0x143, 0xc>(z, v);       // row_bcast:31
    return v;
}

// Exclusive form of an inclusive lane scan (lane 0 gets 0).
template <typename T>
__device__ __forceinline__ T wave_shift_excl(T incl) { return dpp<0x138>(T(0), incl); }  // wave_shr:1

template <typename T, typename Op>
__device__ __forceinline__ T block_reduce(T v, Op op, T *scratch, T id) {
    v = wave_reduce(v, op, id);
    __syncthreads();
    if (lane_id() == 0) scratch[wave_id()] = v;
    __syncthreads();
    T r = scratch[0];
#pragma unroll
    for (int w = 1; w < kWaves; ++w) r = op(r, scratch[w]);
    return r;
}

struct OpMaxF { __device__ float operator()(float a, float b) const { return fmaxf(a, b); } };
struct OpMaxQ {
    __device__ unsigned long long operator()(unsigned long long a, unsigned long long b) const { return a > b ? a : b; }
};
struct OpMinI { __device__ int operator()(int a, int b) const { return a < b ? a : b; } };
struct OpMaxI { __device__ int operator()(int a, int b) const { return a > b ? a : b; } };
struct OpSumI { __device__ int operator()(int a, int b) const { return a + b; } };
struct OpSumD { __device__ double operator()(double a, double b) const { return a + b; } };
struct OpSumQ {
    __device__ unsigned long long operator()(unsigned long long a, unsigned long long b) const { return a + b; }
};
struct OpOrI { __device__ int operator()(int a, int b) const { return a | b; } };
struct OpMinU { __device__ uint32_t operator()(uint32_t a, uint32_t b) const { return a < b ? a : b; } };
struct OpMaxU { __device__ uint32_t operator()(uint32_t a, uint32_t b) const { return a > b ? a : b; } };

__device__ __forceinline__ float block_max(float v, Red &ms) { return block_reduce(v, OpMaxF(), ms.red.f, kNegInf); }
__device__ __forceinline__ int block_min(int v, Red &ms) { return block_reduce(v, OpMinI(), ms.red.i, 0x7fffffff); }
__device__ __forceinline__ int block_maxi(int v, Red &ms) { return block_reduce(v, OpMaxI(), ms.red.i, (int)0x80000000); }
__device__ __forceinline__ int block_sum(int v, Red &ms) { return block_reduce(v, OpSumI(), ms.red.i, 0); }
__device__ __forceinline__ int block_or(int v, Red &ms) { return block_reduce(v, OpOrI(), ms.red.i, 0); }
__device__ __forceinline__ double block_sumd(double v, Red &ms) { return block_reduce(v, OpSumD(), ms.red.d, 0.0); }
__device__ __forceinline__ unsigned long long block_sumq(unsigned long long v, Red &ms) {
    return block_reduce(v, OpSumQ(), ms.red.q, 0ull);
}

// Exclusive scan over the workgroup in thread order; `total` receives the sum.
template <typename T>
__device__ __forceinline__ T block_excl_scan(T v, T *scratch, T &total) {
    const T incl = wave_incl_scan(v);
    const T excl = wave_shift_excl(incl);
    const T wt = readlane(incl, 63);
    __syncthreads();
    if (lane_id() == 0) scratch[wave_id()] = wt;
    __syncthreads();
    T base = T(0), tot = T(0);
#pragma unroll
    for (int w = 0; w < kWaves; ++w) {
        const T s = scratch[w];
        if (w < wave_id()) base += s;
        tot += s;
    }
    total = tot;
    return base + excl;
}

// Slot of the calling lane in an LDS list grown by `counter` (one LDS atomic per
// wave); call it from the lanes that append.
__device__ __forceinline__ int wave_append(int *counter) {
    const unsigned long long bal = __ballot(true);
    const int first = __ffsll((long long)bal) - 1;
    int base = 0;
    if (lane_id() == first) base = atomicAdd(counter, __popcll(bal));
    base = __builtin_amdgcn_readlane(base, first);
    return base + (int)__popcll(bal & ((1ull << lane_id()) - 1ull));
}

// ---------------------------------------------------------------------------------
// Logits loaders: 16-byte vectors of fp32 (4) or bf16 (8) elements.
template <typename TIn> struct Loader;
// The streaming pass reads every logit once: its 16-byte loads are non-temporal.
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
// Fourth word of a raw buffer resource on gfx9-family GPUs (32-bit data format, no
// swizzle); the third word is the range in bytes, stores beyond it are dropped.
constexpr int kBufferRsrcWord3 = 0x00020000;
constexpr int kBufferNonTemporal = 2;   // cache-policy operand of buffer loads: nt
// vec_rsrc (fp32): the same from a buffer resource at byte offset voff + soff (soff
// uniform), non-temporal; positions past the resource's range read 0.
template <> struct Loader<float> {
    static constexpr int VW = 4;
    __device__ static __forceinline__ void vec(const float *p, float *o) {
        const f32x4 v = __builtin_nontemporal_load(reinterpret_cast<const f32x4 *>(p));
        o[0] = v.x; o[1] = v.y; o[2] = v.z; o[3] = v.w;
    }
    __device__ static __forceinline__ void vec_rsrc(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff, float *o) {
        const u32x4 v = __builtin_amdgcn_raw_buffer_load_b128(r, voff, soff, kBufferNonTemporal);
        o[0] = __uint_as_float(v.x); o[1] = __uint_as_float(v.y); o[2] = __uint_as_float(v.z); o[3] = __uint_as_float(v.w);
    }
    __device__ static __forceinline__ float one(const float *p) { return *p; }
};
template <> struct Loader<uint16_t> {
    static constexpr int VW = 8;
    __device__ static __forceinline__ float bf(uint32_t h) { return __uint_as_float(h << 16); }
    __device__ static __forceinline__ void vec(const uint16_t *p, float *o) {
        const u32x4 v = __builtin_nontemporal_load(reinterpret_cast<const u32x4 *>(p));
        o[0] = bf(v.x & 0xffffu); o[1] = bf(v.x >> 16);
        o[2] = bf(v.y & 0xffffu); o[3] = bf(v.y >> 16);
        o[4] = bf(v.z & 0xffffu); o[5] = bf(v.z >> 16);
        o[6] = bf(v.w & 0xffffu); o[7] = bf(v.w >> 16);
    }

    __device__ static __forceinline__ float one(const uint16_t *p) { return bf(*p); }
};

// Count table of the row's history restricted to [c0, c0 + cn): cnt[i - c0].
template <int C>
__device__ __forceinline__ void build_counts(uint32_t *cnt, const Args &a, int row, int c0, int cn) {
    uint4 *c4 = reinterpret_cast<uint4 *>(cnt);
    for (int i = threadIdx.x; i < C / 4; i += kThreads) c4[i] = make_uint4(0u, 0u, 0u, 0u);
    __syncthreads();
    int h0, h1;
    hist_range(a, row, h0, h1);
    // eight independent loads in flight per thread before any LDS atomic
    for (int hb = h0 + (int)threadIdx.x; hb < h1; hb += 8 * kThreads) {
        int id[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const int h = hb + j * kThreads;
            id[j] = (h < h1) ? a.hist_ids[h] : -1;
        }
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const unsigned rel = (unsigned)(id[j] - c0);
            if (id[j] >= 0 && rel < (unsigned)cn) atomicAdd(&cnt[rel], 1u);
        }
    }
    __syncthreads();
}

// Element of chunk c of `row` in final space: penalties from `cnt` (if non-null),
// then division by T for sampled modes that stream in final space.
template <typename TIn>
__device__ __forceinline__ float element_final(const Args &a, const klsample_row_params &p, int row, int i,
                                               const uint32_t *cnt, int c0, bool divide) {
    const TIn *src = reinterpret_cast<const TIn *>(a.logits) + (int64_t)row * a.row_stride;
    float x = Loader<TIn>::one(src + i);
    if (cnt != nullptr) {
        const uint32_t c = cnt[i - c0];
        if (c) x = penalize(x, c, p);
    }
    if (divide) x = __fdiv_rn(x, p.temperature);
    return x;
}

// ---------------------------------------------------------------------------------
// Lower bound on a chunk's K-th largest value.  Each wave takes the Kw-th largest
// (Kw = ceil(K / 4)) of the maxima of 64*G disjoint groups of its own elements (E/G
// consecutive register elements per group): Kw group maxima, hence Kw elements, are at
// or above it.  The chunk bound is the smallest of the four waves' values, so each
// wave has Kw elements at or above it, K in all.  The waves search in parallel, by
// bisection over order-preserving keys with ballots, without barriers.

// Kw-th largest group-maximum key of the calling wave (low 16 key bits zero, so it may
// sit up to 2^-7 relative below the exact value: a few more candidates, eight fewer
// bisection steps).  Wave-uniform.
template <int E, int G>
__device__ __forceinline__ uint32_t wave_group_bound(const float (&x)[E], int Kw) {
    constexpr int GS = E / G;
    uint32_t k[G];
#pragma unroll
    for (int g = 0; g < G; ++g) {
        float mx = kNegInf;
#pragma unroll
        for (int j = 0; j < GS; ++j) mx = fmaxf(mx, x[g * GS + j]);
        k[g] = fkey(mx);
    }
    uint32_t t = 0u;
    for (int bit = 31; bit >= 16; --bit) {
        const uint32_t cand = t | (1u << bit);
        int c = 0;
#pragma unroll
        for (int g = 0; g < G; ++g) c += __popcll(__ballot(k[g] >= cand));
        if (c >= Kw) t = cand;
    }
    return t;
}

template <int E>
__device__ __forceinline__ uint32_t wave_group_bound_dispatch(const float (&x)[E], int G, int Kw) {
    switch (G) {
        case 1: return wave_group_bound<E, 1>(x, Kw);
        case 2: if constexpr (E >= 2) return wave_group_bound<E, 2>(x, Kw); break;
        case 4: if constexpr (E >= 4) return wave_group_bound<E, 4>(x, Kw); break;
        case 8: if constexpr (E >= 8) return wave_group_bound<E, 8>(x, Kw); break;
        default: if constexpr (E >= 16) return wave_group_bound<E, 16>(x, Kw); break;
    }
    return 0u;
}

// Block-wide fallback: the K-th largest of the maxima of kThreads*G disjoint groups
// (E/G consecutive register elements per group), by one wave over keys in LDS.
template <int E, int G>
__device__ __forceinline__ float block_group_bound(const float (&x)[E], int K, uint32_t *keys, ScanMisc &ms) {
    constexpr int GS = E / G;
    constexpr int PER = kThreads * G / 64;   // keys per lane of the counting wave
#pragma unroll
    for (int g = 0; g < G; ++g) {
        float mx = kNegInf;
#pragma unroll
        for (int j = 0; j < GS; ++j) mx = fmaxf(mx, x[g * GS + j]);
        keys[g * kThreads + threadIdx.x] = fkey(mx);
    }
    __syncthreads();
    if (wave_id() == 0) {
        const int lane = lane_id();
        uint32_t t = 0u;
#pragma unroll 1
        for (int bit = 31; bit >= 8; --bit) {
            // re-read the keys every step: the empty asm keeps the compiler from
            // hoisting all of them into registers for the whole kernel
            __asm__ volatile("" ::: "memory");
            const uint32_t cand = t | (1u << bit);
            int c = 0;
#pragma unroll 4
            for (int j = 0; j < PER; ++j) c += __popcll(__ballot(keys[j * 64 + lane] >= cand));
            if (c >= K) t = cand;
        }
        if (lane == 0) ms.bound_key = t;
    }
    __syncthreads();
    return ms.bound_key < 0x00800000u ? kNegInf : fkey_inv(ms.bound_key);
}

template <int E>
__device__ __forceinline__ float block_group_bound_dispatch(const float (&x)[E], int G, int K, uint32_t *keys,
                                                            ScanMisc &ms) {
    switch (G) {
        case 1: return block_group_bound<E, 1>(x, K, keys, ms);
        case 2: if constexpr (E >= 2) return block_group_bound<E, 2>(x, K, keys, ms); break;
        case 4: if constexpr (E >= 4) return block_group_bound<E, 4>(x, K, keys, ms); break;
        case 8: if constexpr (E >= 8) return block_group_bound<E, 8>(x, K, keys, ms); break;
        default: if constexpr (E >= 16) return block_group_bound<E, 16>(x, K, keys, ms); break;
    }
    return kNegInf;
}

// The chunk bound (-inf: keep every element).  Each wave takes its own bound: groups
// start as coarse as 4*Kw groups per wave allow and a wave refines them while fewer
// than Kw hold a finite element (positions past the end of a partial chunk are -inf).
// If a wave is still short of Kw finite groups (a short chunk, masked or massively
// tied scores), one bound over the whole chunk is taken instead.  `keys` holds
// kThreads * min(E, 16) words of LDS.  Ends with a barrier.
template <int E>
__device__ __forceinline__ float chunk_bound(const float (&x)[E], int K, int cn, uint32_t *keys, ScanMisc &ms) {
    constexpr int kMaxG = E < 16 ? E : 16;
    const int Kw = (K + kWaves - 1) / kWaves;
    uint32_t t = 0u;
    if (Kw <= 64 * kMaxG) {
        int G = 1;
        while (G < kMaxG && 64 * G < 4 * Kw) G <<= 1;
        t = wave_group_bound_dispatch<E>(x, G, Kw);
        while (t < 0x00800000u && G < kMaxG) {
            G <<= 1;
            t = wave_group_bound_dispatch<E>(x, G, Kw);
        }
    }
    if (lane_id() == 0) ms.wbound[wave_id()] = t;
    __syncthreads();
    uint32_t b = ms.wbound[0];
#pragma unroll
    for (int w = 1; w < kWaves; ++w) b = min(b, ms.wbound[w]);
    // keys below that of -FLT_MAX stand for -inf (groups without a finite element)
    if (b >= 0x00800000u) return fkey_inv(b);
    if (K > kThreads * kMaxG) return kNegInf;
    int G = 1;
    while (G < kMaxG && G * kThreads < 4 * K) G <<= 1;
    float bound = block_group_bound_dispatch<E>(x, G, K, keys, ms);
    while (bound == kNegInf && G < kMaxG) {
        G <<= 1;
        bound = block_group_bound_dispatch<E>(x, G, K, keys, ms);
    }
    return bound;
}

// ---------------------------------------------------------------------------------
// Radix selection over a row's entries.  A source enumerates (key, index, score)
// for the entries it contains; each thread visits a disjoint subset.

// The row's candidates in their per-chunk slots: chunk c holds cnt[c] entries (cnt in
// LDS).  Waves take chunks round robin and lanes a chunk's entries, eight loads in
// flight per lane (addresses clamped into the chunk's entries rather than predicated),
// so a chunk of up to 512 candidates is one round trip.
struct CandSource {
    const Cand *cands;
    const int *cnt;
    int S, cap;
    float lo;
    template <class F>
    __device__ __forceinline__ void each(F f) const {
        const int lane = lane_id();
        for (int c = wave_id(); c < S; c += kWaves) {
            const int n = cnt[c];
            const uint2 *p = reinterpret_cast<const uint2 *>(cands + (size_t)c * cap);
            for (int j0 = 0; j0 < n; j0 += 64 * 8) {
                uint2 e[8];
#pragma unroll
                for (int u = 0; u < 8; ++u) e[u] = p[min(j0 + u * 64 + lane, n - 1)];
#pragma unroll
                for (int u = 0; u < 8; ++u) {
                    const float y = __uint_as_float(e[u].x);
                    if (j0 + u * 64 + lane < n && y >= lo) f(fkey(y), (int)e[u].y, y);
                }
            }
        }
    }
};

// n sort keys (desc_key) held in LDS.
struct LdsSource {
    const unsigned long long *sb;
    int n;
    template <class F>
    __device__ __forceinline__ void each(F f) const {
        for (int i = threadIdx.x; i < n; i += kThreads) {
            const unsigned long long k = sb[i];
            const uint32_t key = ~(uint32_t)(k >> 32);
            f(key, (int)(uint32_t)k, fkey_inv(key));
        }
    }
};

// Dense row in final space; an entry is included when its score is above `cut`, or
// equal to it with index <= cut_idx (cut = -inf, cut_idx = V includes everything).
struct DenseSource {
    const float *y;
    int V;
    float cut;
    int cut_idx;
    __device__ __forceinline__ bool keep(float v, int i) const { return v > cut || (v == cut && i <= cut_idx); }
    // Calls f(key, index, score) for every kept entry.  y is 16-byte aligned and
    // readable up to V rounded up to 4.  Blocks of eight 16-byte loads per thread: the
    // next block is requested before the current one is visited (addresses clamped, so
    // the request past the end is a harmless re-read), sixteen loads in flight.
    template <class F>
    __device__ __forceinline__ void each(F f) const {
        constexpr int U = 8;
        constexpr int kStep = kThreads * 4 * U;
        const int vlast = (V - 1) & ~3;
        float4 qa[U], qb[U];
        auto request = [&](float4 (&q)[U], int t0) {
#pragma unroll
            for (int u = 0; u < U; ++u)
                q[u] = *reinterpret_cast<const float4 *>(y + min(t0 + (u * kThreads + (int)threadIdx.x) * 4, vlast));
        };
        request(qa, 0);
        for (int t0 = 0; t0 < V; t0 += kStep) {
            request(qb, t0 + kStep);
#pragma unroll
            for (int u = 0; u < U; ++u) {
                const int i = t0 + (u * kThreads + (int)threadIdx.x) * 4;
                const float v4[4] = {qa[u].x, qa[u].y, qa[u].z, qa[u].w};
#pragma unroll
                for (int e = 0; e < 4; ++e)
                    if (i + e < V && keep(v4[e], i + e)) f(fkey(v4[e]), i + e, v4[e]);
            }
#pragma unroll
            for (int u = 0; u < U; ++u) qa[u] = qb[u];
        }
    }
};

// Wave 0 scans 256 histogram bins from the highest digit down and records the
// first bin at which the running count reaches `need`.
__device__ __forceinline__ void pick_digit_count(Misc &ms, uint32_t need) {
    if (threadIdx.x < 64) {
        const int l = lane_id();
        uint32_t c[4], s = 0;
#pragma unroll
        for (int j = 0; j < 4; ++j) { c[j] = ms.hist[255 - 4 * l - j]; s += c[j]; }
        const uint32_t incl = wave_incl_scan(s);
        const uint32_t excl = incl - s;
        const unsigned long long bal = __ballot(incl >= need);
        const int first = bal ? (__ffsll((long long)bal) - 1) : 63;
        if (l == first) {
            uint32_t acc = excl;
            int digit = 255 - 4 * l - 3;
            uint32_t rem = need > acc ? need - acc : 1u;
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                if (acc + c[j] >= need) { digit = 255 - 4 * l - j; rem = need - acc; break; }
                acc += c[j];
            }
            ms.sel_digit = (uint32_t)digit;
            ms.sel_need = rem;
        }
    }
    __syncthreads();
}

// Key of the R-th largest entry of `src` (R >= 1, R <= number of entries).
template <typename Src>
__device__ __forceinline__ uint32_t select_kth(const Src &src, uint32_t R, Misc &ms) {
    uint32_t prefix = 0u, need = R;
    for (int shift = 24; shift >= 0; shift -= 8) {
        const uint32_t hmask = (shift == 24) ? 0u : (0xffffffffu << (shift + 8));
        for (int i = threadIdx.x; i < 256; i += kThreads) ms.hist[i] = 0u;
        __syncthreads();
        src.each([&](uint32_t key, int, float) {
            if ((key & hmask) == prefix) atomicAdd(&ms.hist[(key >> shift) & 255u], 1u);
        });
        __syncthreads();
        pick_digit_count(ms, need);
        prefix |= ms.sel_digit << shift;
        need = ms.sel_need;
        __syncthreads();
    }
    return prefix;
}

// Mass-weighted selection: walking entries from the largest score down in groups of
// equal score, find the first group g whose cumulative fixed-point mass (all groups
// above g plus g itself) exceeds `target`.  Returns false if the total does not.
struct MassPick {
    uint32_t key;                  // key of group g
    unsigned long long above;      // mass of all entries above g
    uint32_t above_count;          // entries above g
    uint32_t group_count;          // entries in g
    unsigned long long group_mass; // mass of g
};

template <typename Src>
__device__ __forceinline__ bool select_mass(const Src &src, double target, float m, MassPick &out, Misc &ms) {
    uint32_t prefix = 0u;
    unsigned long long above = 0ull;
    uint32_t above_count = 0u;
    for (int shift = 24; shift >= 0; shift -= 8) {
        const uint32_t hmask = (shift == 24) ? 0u : (0xffffffffu << (shift + 8));
        for (int i = threadIdx.x; i < 256; i += kThreads) { ms.hist[i] = 0u; ms.hmass[i] = 0ull; }
        __syncthreads();
        src.each([&](uint32_t key, int, float v) {
            if ((key & hmask) == prefix) {
                const uint32_t b = (key >> shift) & 255u;
                atomicAdd(&ms.hist[b], 1u);
                atomicAdd(&ms.hmass[b], weight_fix(v, m));
            }
        });
        __syncthreads();
        if (threadIdx.x < 64) {
            const int l = lane_id();
            unsigned long long c[4], s = 0ull;
            uint32_t n[4], ns = 0u;
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                c[j] = ms.hmass[255 - 4 * l - j]; s += c[j];
                n[j] = ms.hist[255 - 4 * l - j]; ns += n[j];
            }
            const unsigned long long incl = wave_incl_scan(s);
            const uint32_t nincl = wave_incl_scan(ns);
            const unsigned long long bal = __ballot((double)(above + incl) > target);
            if (bal == 0ull) {
                if (l == 0) ms.sel_found = 0;
            } else if (l == __ffsll((long long)bal) - 1) {
                unsigned long long acc = above + (incl - s);
                uint32_t nacc = above_count + (nincl - ns);
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    if ((double)(acc + c[j]) > target) {
                        ms.sel_digit = (uint32_t)(255 - 4 * l - j);
                        ms.sel_above_mass = acc;
                        ms.sel_above_count = nacc;
                        ms.sel_need = n[j];
                        ms.hmass[0] = c[j];  // group mass at the final level (read below)
                        break;
                    }
                    acc += c[j];
                    nacc += n[j];
                }
                ms.sel_found = 1;
            }
        }
        __syncthreads();
        if (!ms.sel_found) { __syncthreads(); return false; }
        prefix |= ms.sel_digit << shift;
        above = ms.sel_above_mass;
        above_count = ms.sel_above_count;
        out.group_count = ms.sel_need;
        out.group_mass = ms.hmass[0];
        __syncthreads();
    }
    out.key = prefix;
    out.above = above;
    out.above_count = above_count;
    return true;
}

// Walk items [0, n) in order; `weight(i)` >= 0 (a pure function of i).  Returns the
// first item whose inclusive cumulative weight exceeds `target`, or -1; `last`
// receives the last item with positive weight (-1 if none) and `before` the weight
// before the returned item (the total if none).  Three steps: per-segment sums (one
// wave per segment, lanes strided, eight weights in flight per lane), the crossing
// segment (one wave scan), and inside it runs of eight items per lane.
template <typename W>
__device__ __forceinline__ int ordered_find(int n, W weight, double target, Misc &ms, int &last, double &before) {
    int seg = 2048;
    while ((n + seg - 1) / seg > kSegCap) seg *= 2;
    const int nseg = (n + seg - 1) / seg;
    const int lane = lane_id();
    if (nseg <= 1) {
        // one segment: the run walk alone
        if (wave_id() == 0) {
            double base = 0.0, bf = 0.0;
            int found = -1, lastp = -1;
            for (int r0 = 0; r0 < n && found < 0; r0 += 64 * 8) {
                const int l0 = r0 + 8 * lane;
                double wv[8], ls = 0.0;
                int lp = -1;
#pragma unroll
                for (int j = 0; j < 8; ++j) {
                    const double x = weight(min(l0 + j, n - 1));
                    wv[j] = (l0 + j < n) ? x : 0.0;
                    ls += wv[j];
                    if (wv[j] > 0.0) lp = l0 + j;
                }
                lastp = max(lastp, wave_reduce(lp, OpMaxI(), -1));
                const double incl = wave_incl_scan(ls);
                const double ex = wave_shift_excl(incl);
                const unsigned long long bal = __ballot(base + ex + ls > target);
                if (bal != 0ull) {
                    const int fl = __ffsll((long long)bal) - 1;
                    int f = -1;
                    double c = base + ex, cb = 0.0;
                    if (lane == fl) {
                        int lpos = -1;
#pragma unroll
                        for (int j = 0; j < 8; ++j) {
                            if (wv[j] > 0.0) {
                                if (f < 0 && c + wv[j] > target) { f = l0 + j; cb = c; }
                                if (f < 0) c += wv[j];
                                lpos = l0 + j;
                            }
                        }
                        if (f < 0) { f = lpos; cb = c; }
                    }
                    found = readlane(f, fl);
                    bf = readlane(cb, fl);
                } else {
                    base += readlane(incl, 63);
                }
            }
            if (lane == 0) { ms.ib = found; ms.db = found < 0 ? base : bf; ms.last = lastp; }
        }
        __syncthreads();
        const int found = ms.ib;
        before = ms.db;
        last = ms.last;
        __syncthreads();
        return found;
    }
    for (int sg = wave_id(); sg < nseg; sg += kWaves) {
        const int b0 = sg * seg, b1 = min(n, b0 + seg);
        double sum = 0.0;
        int lp = -1;
        for (int i0 = b0; i0 < b1; i0 += 64 * 8) {
            double wv[8];
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                const int i = i0 + j * 64 + lane;
                const double x = weight(min(i, b1 - 1));
                wv[j] = (i < b1) ? x : 0.0;
            }
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                sum += wv[j];
                if (wv[j] > 0.0) lp = i0 + j * 64 + lane;
            }
        }
        sum = wave_reduce(sum, OpSumD(), 0.0);
        lp = wave_reduce(lp, OpMaxI(), -1);
        if (lane == 0) { ms.seg[sg] = sum; ms.segl[sg] = lp; }
    }
    __syncthreads();
    if (wave_id() == 0) {
        const int s0 = 2 * lane, s1 = 2 * lane + 1;
        const double a0 = s0 < nseg ? ms.seg[s0] : 0.0, a1 = s1 < nseg ? ms.seg[s1] : 0.0;
        const int lp = max(s0 < nseg ? ms.segl[s0] : -1, s1 < nseg ? ms.segl[s1] : -1);
        const double incl = wave_incl_scan(a0 + a1);
        const double ex = wave_shift_excl(incl);
        const bool c0 = s0 < nseg && ex + a0 > target;
        const bool c1 = s1 < nseg && (ex + a0) + a1 > target;
        const unsigned long long bal = __ballot(c0 || c1);
        const int lpm = wave_reduce(lp, OpMaxI(), -1);
        if (bal == 0ull) {
            if (lane == 0) { ms.ia = -1; ms.da = 0.0; }
            if (lane == 63) ms.db = incl;
        } else if (lane == __ffsll((long long)bal) - 1) {
            ms.ia = c0 ? s0 : s1;
            ms.da = c0 ? ex : ex + a0;
        }
        if (lane == 0) ms.last = lpm;
    }
    __syncthreads();
    const int sg = ms.ia;
    last = ms.last;
    if (sg < 0) {
        before = ms.db;
        __syncthreads();
        return -1;
    }
    if (wave_id() == 0) {
        const int b0 = sg * seg, b1 = min(n, b0 + seg);
        double base = ms.da;
        int found = -1;
        double bf = 0.0;
        for (int r0 = b0; r0 < b1 && found < 0; r0 += 64 * 8) {
            const int l0 = r0 + 8 * lane;
            double wv[8], ls = 0.0;
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                const double x = weight(min(l0 + j, b1 - 1));
                wv[j] = (l0 + j < b1) ? x : 0.0;
                ls += wv[j];
            }
            const double incl = wave_incl_scan(ls);
            const double ex = wave_shift_excl(incl);
            const unsigned long long bal = __ballot(base + ex + ls > target);
            if (bal != 0ull) {
                const int fl = __ffsll((long long)bal) - 1;
                int f = -1;
                double c = base + ex, cb = 0.0;
                if (lane == fl) {
                    int lpos = -1;
#pragma unroll
                    for (int j = 0; j < 8; ++j) {
                        if (wv[j] > 0.0) {
                            if (f < 0 && c + wv[j] > target) { f = l0 + j; cb = c; }
                            if (f < 0) c += wv[j];
                            lpos = l0 + j;
                        }
                    }
                    if (f < 0) { f = lpos; cb = c; }   // rounding: the run's sum crossed, its items did not
                }
                found = readlane(f, fl);
                bf = readlane(cb, fl);
            } else {
                base += readlane(incl, 63);
            }
        }
        if (found < 0) { found = ms.segl[sg]; bf = base; }   // rounding: no item of the segment crossed
        if (lane == 0) { ms.ib = found; ms.db = bf; }
    }
    __syncthreads();
    const int found = ms.ib;
    before = ms.db;
    __syncthreads();
    return found;
}

// Inverse CDF over a dense source in vocab order: the first kept entry whose inclusive
// cumulative weight_fix(y, m) exceeds `target` (same fixed point), or -1; `last`
// receives the last kept entry of positive weight (-1 if none).  Segments of
// kDrawStep * g consecutive entries (at most kSegCap of them), one wave per segment:
// segment sums from 16-byte loads, the wave's next step requested before the current
// one is summed; then wave 0 finds the crossing segment and walks it.  The sums are
// integers, exact and independent of their order, so the crossing segment holds the
// crossing entry.
constexpr int kDrawStep = 64 * 4 * 8;   // entries per wave step: eight 16-byte loads per lane

__device__ __forceinline__ int dense_draw(const DenseSource &src, float m, unsigned long long target, Misc &ms,
                                          int &last) {
    const int V = src.V;
    int g = 1;
    while ((V + kDrawStep * g - 1) / (kDrawStep * g) > kSegCap) g <<= 1;
    const int seg = kDrawStep * g;
    const int nseg = (V + seg - 1) / seg;
    const int lane = lane_id(), w = wave_id();
    const int vlast = (V - 1) & ~3;
    unsigned long long *segq = reinterpret_cast<unsigned long long *>(ms.seg);
    auto request = [&](float4 (&q)[8], int base) {
#pragma unroll
        for (int u = 0; u < 8; ++u) q[u] = *reinterpret_cast<const float4 *>(src.y + min(base + (u * 64 + lane) * 4, vlast));
    };
    auto weight = [&](float v, int i) -> unsigned long long {
        return (i < V && src.keep(v, i)) ? weight_fix(v, m) : 0ull;
    };
    // 1. segment sums: wave w takes segments w, w + kWaves, ... step by step
    const int nsteps = ((nseg - w + kWaves - 1) / kWaves) * g;
    auto step_base = [&](int k) { return (w + kWaves * (k / g)) * seg + (k % g) * kDrawStep; };
    float4 qa[8], qb[8];
    request(qa, step_base(0));
    unsigned long long sum = 0ull;
    int lp = -1;
    for (int k = 0; k < nsteps; ++k) {
        request(qb, step_base(min(k + 1, nsteps - 1)));
        const int b = step_base(k);
#pragma unroll
        for (int u = 0; u < 8; ++u) {
            const int i0 = b + (u * 64 + lane) * 4;
            const float v4[4] = {qa[u].x, qa[u].y, qa[u].z, qa[u].w};
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const unsigned long long wt = weight(v4[e], i0 + e);
                sum += wt;
                if (wt) lp = i0 + e;
            }
        }
        if (k % g == g - 1) {
            sum = wave_reduce(sum, OpSumQ(), 0ull);
            lp = wave_reduce(lp, OpMaxI(), -1);
            if (lane == 0) { segq[w + kWaves * (k / g)] = sum; ms.segl[w + kWaves * (k / g)] = lp; }
            sum = 0ull;
            lp = -1;
        }
#pragma unroll
        for (int u = 0; u < 8; ++u) qa[u] = qb[u];
    }
    __syncthreads();
    // 2. the crossing segment (two per lane)
    if (w == 0) {
        const int s0 = 2 * lane, s1 = 2 * lane + 1;
        const unsigned long long a0 = s0 < nseg ? segq[s0] : 0ull, a1 = s1 < nseg ? segq[s1] : 0ull;
        const int l2 = max(s0 < nseg ? ms.segl[s0] : -1, s1 < nseg ? ms.segl[s1] : -1);
        const unsigned long long incl = wave_incl_scan(a0 + a1);
        const unsigned long long ex = incl - (a0 + a1);
        const bool c0 = s0 < nseg && ex + a0 > target;
        const bool c1 = s1 < nseg && ex + a0 + a1 > target;
        const unsigned long long bal = __ballot(c0 || c1);
        const int lpm = wave_reduce(l2, OpMaxI(), -1);
        if (bal == 0ull) {
            if (lane == 0) ms.ia = -1;
        } else if (lane == __ffsll((long long)bal) - 1) {
            ms.ia = c0 ? s0 : s1;
            ms.sel_above_mass = c0 ? ex : ex + a0;
        }
        if (lane == 0) ms.last = lpm;
    }
    __syncthreads();
    const int sg = ms.ia;
    last = ms.last;
    // 3. its walk, one step (eight loads per lane) at a time
    if (w == 0 && sg >= 0) {
        unsigned long long run = ms.sel_above_mass;
        int found = -1;
        for (int k = 0; k < g && found < 0; ++k) {
            const int b = sg * seg + k * kDrawStep;
            request(qa, b);
#pragma unroll
            for (int u = 0; u < 8; ++u) {
                if (found >= 0) break;
                const int i0 = b + (u * 64 + lane) * 4;
                const float v4[4] = {qa[u].x, qa[u].y, qa[u].z, qa[u].w};
                unsigned long long wv[4], ls = 0ull;
#pragma unroll
                for (int e = 0; e < 4; ++e) { wv[e] = weight(v4[e], i0 + e); ls += wv[e]; }
                const unsigned long long incl = run + wave_incl_scan(ls);
                const unsigned long long bal = __ballot(incl > target);
                if (bal != 0ull) {
                    const int fl = __ffsll((long long)bal) - 1;
                    int f = -1;
                    if (lane == fl) {
                        unsigned long long c = incl - ls;
#pragma unroll
                        for (int e = 0; e < 4; ++e) {
                            if (f < 0 && c + wv[e] > target) f = i0 + e;
                            c += wv[e];
                        }
                    }
                    found = readlane(f, fl);
                } else {
                    run = readlane(incl, 63);
                }
            }
        }
        if (found < 0) found = ms.segl[sg];
        if (lane == 0) ms.ib = found;
    }
    __syncthreads();
    const int found = sg >= 0 ? ms.ib : -1;
    __syncthreads();
    return found;
}

// Bitonic sort (ascending) of n = power of two 64-bit keys in LDS.
__device__ __forceinline__ void bitonic_sort(unsigned long long *s, int n) {
    for (int k = 2; k <= n; k <<= 1) {
        for (int j = k >> 1; j > 0; j >>= 1) {
            for (int i = threadIdx.x; i < n; i += kThreads) {
                const int l = i ^ j;
                if (l > i) {
                    const unsigned long long x = s[i], y = s[l];
                    const bool up = (i & k) == 0;
                    if ((x > y) == up) { s[i] = y; s[l] = x; }
                }
            }
            __syncthreads();
        }
    }
}

__device__ __forceinline__ int pow2_ceil(int n) {
    int p = 1;
    while (p < n) p <<= 1;
    return p;
}

// A chunk summary as two 16-byte loads (one request per half, never split or predicated).
__device__ __forceinline__ ChunkStat load_stat(const ChunkStat *p) {
    const uint4 *q = reinterpret_cast<const uint4 *>(p);
    const uint4 u = q[0], v = q[1];
    ChunkStat s;
    s.m = __uint_as_float(u.x);
    s.arg = (int32_t)u.y;
    s.y_thr = __uint_as_float(u.z);
    s.ncand = (int32_t)u.w;
    s.z = __hiloint2double((int)v.y, (int)v.x);
    s.flags = (int32_t)v.z;
    s.nfinite = (int32_t)v.w;
    return s;
}

// Sort key: ascending order = score descending, then index ascending.
__device__ __forceinline__ unsigned long long desc_key(float y, int idx) {
    return ((unsigned long long)(~fkey(y)) << 32) | (uint32_t)idx;
}
__device__ __forceinline__ float desc_key_y(unsigned long long k) { return fkey_inv(~(uint32_t)(k >> 32)); }
__device__ __forceinline__ int desc_key_idx(unsigned long long k) { return (int)(uint32_t)k; }


// Sort sb[0..n) (distinct keys, 2 <= n <= kThreads) ascending with the whole block:
// the kThreads / n threads given to a key each count the keys below it in one slice of
// sb (broadcast 16-byte reads), and the slices' counts are added.  `part` holds
// kThreads ints of LDS.  Three barriers.
__device__ __forceinline__ void block_rank_sort(unsigned long long *sb, int n, uint32_t *part) {
    const int tid = threadIdx.x;
    const int segs = kThreads / n;
    const int k = tid % n, sg = tid / n;
    const int len = (((n + segs - 1) / segs) + 1) & ~1;   // even: slices start 16-byte aligned
    unsigned long long key = ~0ull;
    uint32_t cnt = 0u;
    if (sg < segs) {
        key = sb[k];
        const int j0 = sg * len, j1 = min(n, j0 + len);
#pragma unroll 4
        for (int j = j0; j < j1; j += 2) {
            const ulonglong2 q = *reinterpret_cast<const ulonglong2 *>(&sb[j]);
            cnt += (q.x < key) ? 1u : 0u;
            cnt += (j + 1 < j1 && q.y < key) ? 1u : 0u;
        }
    }
    part[tid] = cnt;
    __syncthreads();
    int rank = 0;
    if (tid < n)
        for (int g = 0; g < segs; ++g) rank += (int)part[g * n + tid];
    __syncthreads();
    if (tid < n) sb[rank] = key;
    __syncthreads();
}

// Vocab-order ranks of the entries D[0..L) (1 <= L <= 64, distinct indices) into
// irank[0..L), counted by the whole block as in block_rank_sort.  Two barriers.
__device__ __forceinline__ void block_index_rank(const unsigned long long *D, int L, uint32_t *part, uint32_t *irank) {
    const int tid = threadIdx.x;
    const int segs = kThreads / L;
    const int k = tid % L, sg = tid / L;
    const int len = (((L + segs - 1) / segs) + 1) & ~1;
    uint32_t cnt = 0u;
    if (sg < segs) {
        const int mine = desc_key_idx(D[k]);
        const int j0 = sg * len, j1 = min(L, j0 + len);
        for (int j = j0; j < j1; j += 2) {
            const ulonglong2 q = *reinterpret_cast<const ulonglong2 *>(&D[j]);
            cnt += (desc_key_idx(q.x) < mine) ? 1u : 0u;
            cnt += (j + 1 < j1 && desc_key_idx(q.y) < mine) ? 1u : 0u;
        }
    }
    part[tid] = cnt;
    __syncthreads();
    if (tid < L) {
        uint32_t r = 0u;
        for (int g = 0; g < segs; ++g) r += part[g * L + tid];
        irank[tid] = r;
    }
    __syncthreads();
}

// Sorts in[0..n) (2 <= n <= 64, distinct keys and indices) ascending into out, and
// records at each sorted position the entry's rank in vocab order among all n
// (irank).  Value and index comparisons share one pass of the whole block (the two
// counts packed in one word); two barriers.
__device__ __forceinline__ void block_rank_sort_idx(const unsigned long long *in, int n, unsigned long long *out,
                                                    uint32_t *part, uint32_t *irank) {
    const int tid = threadIdx.x;
    const int segs = kThreads / n;
    const int k = tid % n, sg = tid / n;
    const int len = (((n + segs - 1) / segs) + 1) & ~1;
    unsigned long long key = ~0ull;
    uint32_t cnt = 0u;
    if (sg < segs) {
        key = in[k];
        const int mine = desc_key_idx(key);
        const int j0 = sg * len, j1 = min(n, j0 + len);
        for (int j = j0; j < j1; j += 2) {
            const ulonglong2 q = *reinterpret_cast<const ulonglong2 *>(&in[j]);
            cnt += ((q.x < key) ? 1u : 0u) + ((desc_key_idx(q.x) < mine) ? 65536u : 0u);
            if (j + 1 < j1) cnt += ((q.y < key) ? 1u : 0u) + ((desc_key_idx(q.y) < mine) ? 65536u : 0u);
        }
    }
    part[tid] = cnt;
    __syncthreads();
    if (tid < n) {
        uint32_t r = 0u;
        for (int g = 0; g < segs; ++g) r += part[g * n + tid];
        out[r & 0xffffu] = key;
        irank[r & 0xffffu] = r >> 16;
    }
    __syncthreads();
}

// Sort n distinct keys ascending in LDS (capacity >= pow2_ceil(n)).
__device__ __forceinline__ void sort_keys(unsigned long long *sb, int n, uint32_t *part) {
    if (n <= 1) return;
    if (n <= kThreads) {
        block_rank_sort(sb, n, part);
        return;
    }
    const int n2 = pow2_ceil(n);
    for (int i = n + (int)threadIdx.x; i < n2; i += kThreads) sb[i] = ~0ull;
    __syncthreads();
    bitonic_sort(sb, n2);
}

// ---------------------------------------------------------------------------------
// Outputs of a resolved row.

// With hist_append (history ranges as begin/end pairs), the row's token is also stored
// just past its history, so the caller's next range is one longer.
__device__ __forceinline__ void append_token(const Args &a, int row, int token) {
    if (a.hist_append == nullptr) return;
    int h0, h1;
    hist_range(a, row, h0, h1);
    a.hist_append[h1] = token;
}

struct RowOut {
    int token;
    double logprob;
    float m;          // max final score
    float cut;        // smallest kept score
    int cut_idx;      // largest kept index among scores equal to `cut`
    int kept;
    double log_norm;  // log of the kept mass relative to exp(m)
    int path;
};

// Thread 0 writes token / logprob / row state; all threads write the top-N list
// from ms.topn_* (`count` finite entries, best first).  Slots from `count` up to
// min(N, V) are -inf entries whose ids are the smallest not already listed;
// slots beyond min(N, V) (only when V < N) hold id -1.
__device__ __forceinline__ void write_row(const Args &a, int row, int mode, const RowOut &r, int count, Misc &ms) {
    const int N = a.N, V = a.V;
    if (N > 0) {
        const int nv = min(N, V);
        int32_t *ids = a.top_ids + (size_t)row * N;
        float *lps = a.top_lp + (size_t)row * N;
        for (int t = threadIdx.x; t < N; t += kThreads) {
            if (t < count && t < nv) {
                ids[t] = ms.topn_idx[t];
                lps[t] = (float)((double)ms.topn_y[t] - (double)r.m - r.log_norm);
            } else if (t >= nv) {
                ids[t] = -1;
                lps[t] = kNegInf;
            }
        }
        if (count < nv) {
            // the answer lies in [0, count + nv) <= [0, 2N): a bitmap of listed ids
            uint32_t *bm = ms.hist;
            __syncthreads();
            for (int i = threadIdx.x; i < 256; i += kThreads) bm[i] = 0u;
            __syncthreads();
            for (int t = threadIdx.x; t < count; t += kThreads) {
                const int id = ms.topn_idx[t];
                if (id < 2 * kMaxLogprobs) atomicOr(&bm[id >> 5], 1u << (id & 31));
            }
            __syncthreads();
            if (threadIdx.x == 0) {
                int j = 0;
                for (int t = count; t < nv; ++t) {
                    while ((bm[j >> 5] >> (j & 31)) & 1u) ++j;
                    ids[t] = j;
                    lps[t] = kNegInf;
                    ++j;
                }
            }
        }
    }
    if (threadIdx.x == 0) {
        a.token[row] = r.token;
        append_token(a, row, r.token);
        a.logprob[row] = (float)r.logprob;
        klsample_row_info info;
        info.max_score = r.m;
        info.cut_score = r.cut;
        info.cut_index = r.cut_idx;
        info.kept = r.kept;
        info.log_norm = r.log_norm;
        info.path = r.path;
        info.mode = mode;
        a.rows[row] = info;
        if (a.row_info) a.row_info[row] = info;
    }
}

// Top-N of the entries of a dense source, best first, into ms.topn_*; ties at the
// N-th score are taken in index order.  Returns the number written.
__device__ __forceinline__ int dense_topn(const DenseSource &src, int N, unsigned long long *sortbuf, Misc &ms) {
    if (N <= 0) return 0;
    int total = 0;
    src.each([&](uint32_t, int, float) { ++total; });
    total = block_sum(total, ms);
    const int want = min(N, total);
    if (want == 0) return 0;
    const uint32_t kN = select_kth(src, (uint32_t)want, ms);
    if (threadIdx.x == 0) ms.ncand = 0;
    __syncthreads();
    src.each([&](uint32_t key, int idx, float y) {
        if (key > kN) {
            const int pos = atomicAdd(&ms.ncand, 1);
            ms.topn_idx[pos] = idx;
            ms.topn_y[pos] = y;
        }
    });
    __syncthreads();
    const int ngt = ms.ncand;
    const int need = want - ngt;
    const float tauN = fkey_inv(kN);
    int base = 0;
    for (int t0 = 0; t0 < src.V && base < need; t0 += kThreads * 4) {
        const int i0 = t0 + 4 * (int)threadIdx.x;
        int f[4], s = 0;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int i = i0 + j;
            f[j] = 0;
            if (i < src.V) {
                const float v = src.y[i];
                f[j] = (fkey(v) == kN && src.keep(v, i)) ? 1 : 0;
            }
            s += f[j];
        }
        int tot;
        int rank = base + block_excl_scan(s, ms.red.i, tot);
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            if (f[j]) {
                if (rank < need) { ms.topn_idx[ngt + rank] = i0 + j; ms.topn_y[ngt + rank] = tauN; }
                ++rank;
            }
        }
        base += tot;
    }
    __syncthreads();
    const int n2 = pow2_ceil(want);
    for (int i = threadIdx.x; i < n2; i += kThreads)
        sortbuf[i] = (i < want) ? desc_key(ms.topn_y[i], ms.topn_idx[i]) : ~0ull;
    __syncthreads();
    bitonic_sort(sortbuf, n2);
    for (int i = threadIdx.x; i < want; i += kThreads) {
        ms.topn_idx[i] = desc_key_idx(sortbuf[i]);
        ms.topn_y[i] = desc_key_y(sortbuf[i]);
    }
    __syncthreads();
    return want;
}

// Top-p cut inside a sorted run of entries: G[0..n) (n >= 1) sorted best first, every
// entry scoring above them already counted (`above` fixed-point mass, `above_count`
// entries).  Walking from the top, the first entry whose inclusive mass exceeds
// `target` crosses; of its group of equal scores, entries are kept in index order while
// their exclusive mass does not exceed `target` (at least one).  If no entry crosses
// (rounding), the last entry is taken as the crossing one.  All threads receive the
// result.
__device__ __forceinline__ void cut_in_sorted(const unsigned long long *G, int n, unsigned long long above,
                                              uint32_t above_count, double target, float m, TopPCut &out, Misc &ms) {
    if (wave_id() == 0) {
        const int l = lane_id();
        unsigned long long run = above;
        int j = -1;
        unsigned long long incl_j = 0ull;
        for (int i0 = 0; i0 < n && j < 0; i0 += 64) {
            const int i = i0 + l;
            const unsigned long long w = i < n ? weight_fix(desc_key_y(G[i]), m) : 0ull;
            const unsigned long long incl = run + wave_incl_scan(w);
            const unsigned long long bal = __ballot(i < n && (double)incl > target);
            if (bal != 0ull) {
                const int fl = __ffsll((long long)bal) - 1;
                j = i0 + fl;
                incl_j = readlane(incl, fl);
            }
            run = readlane(incl, 63);
        }
        if (j < 0) j = n - 1, incl_j = run;   // rounding: take the last entry
        // the group of equal scores around j: [gs, ge)
        const float yg = desc_key_y(G[j]);
        const unsigned long long kg = (unsigned long long)(~fkey(yg)) << 32;
        int lo = 0, hi = j;
        while (lo < hi) { const int mid = (lo + hi) >> 1; if (G[mid] < kg) lo = mid + 1; else hi = mid; }
        const int gs = lo;
        lo = j + 1; hi = n;
        while (lo < hi) { const int mid = (lo + hi) >> 1; if ((G[mid] >> 32) == (kg >> 32)) lo = mid + 1; else hi = mid; }
        const int ge = lo;
        const unsigned long long wt = weight_fix(yg, m);
        const unsigned long long above_g = incl_j - (unsigned long long)(j - gs + 1) * wt;
        const int count = ge - gs;
        int keep = count;
        if (wt > 0ull) {
            const double room = target - (double)above_g;
            const double k = floor(room / (double)wt) + 1.0;
            keep = (int)fmin((double)count, fmax(1.0, k));
        }
        if (l == 0) {
            TopPCut r;
            r.cut = yg;
            r.cut_idx = (keep < count) ? desc_key_idx(G[gs + keep - 1]) : 0x7fffffff;
            r.kept = (int)above_count + gs + keep;
            r.zf = above_g + (unsigned long long)keep * wt;
            ms.topp = r;
        }
    }
    __syncthreads();
    out = ms.topp;
    __syncthreads();
}

// Top-p cut over a dense source by a mass histogram in log space: bin b holds the
// kept entries with (m - y) * 64 in [b, b + 1) (the last bin everything further
// down), which orders bins like scores.  The bin where the running mass from the top
// first exceeds `target` is gathered into LDS, sorted, and walked to the first group
// of equal scores whose mass crosses; ties in that group are kept in index order as
// far as the remaining mass allows.  Returns 1 with the cut, 0 if the whole source's
// mass does not exceed `target` (everything kept), -1 if the bin is the last one or
// too large for LDS (the caller falls back to the radix selection).  zk / nk receive
// the source's total mass and finite count either way (except -1).
constexpr int kMassBins = 2048;

__device__ __forceinline__ int topp_cut_bins(const DenseSource &src, float m, float top_p, unsigned char *raw,
                                             int cap, unsigned long long &zk, int &nk, TopPCut &out, Misc &ms) {
    uint32_t *hn = reinterpret_cast<uint32_t *>(raw);
    unsigned long long *hw = reinterpret_cast<unsigned long long *>(raw + kMassBins * 4);
    for (int i = threadIdx.x; i < kMassBins; i += kThreads) { hn[i] = 0u; hw[i] = 0ull; }
    if (threadIdx.x == 0) { ms.ncand = 0; ms.flag = 0; }
    __syncthreads();
    auto bin = [m](float y) -> int {
        const float d = (m - y) * 64.0f;
        return d < (float)(kMassBins - 1) ? (int)d : kMassBins - 1;
    };
    src.each([&](uint32_t, int, float y) {
        if (y > kNegInf) {
            const int b = bin(y);
            atomicAdd(&hn[b], 1u);
            atomicAdd(&hw[b], weight_fix(y, m));
        }
    });
    __syncthreads();
    if (wave_id() == 0) {
        // 32 consecutive bins per lane
        const int l = lane_id();
        unsigned long long ws = 0ull;
        uint32_t cs = 0u;
#pragma unroll 8
        for (int j = 0; j < kMassBins / 64; ++j) { ws += hw[l * (kMassBins / 64) + j]; cs += hn[l * (kMassBins / 64) + j]; }
        const unsigned long long wi = wave_incl_scan(ws);
        const uint32_t ci = wave_incl_scan(cs);
        const unsigned long long total = readlane(wi, 63);
        const double target = (double)top_p * (double)total;
        const unsigned long long bal = __ballot((double)wi > target);
        const uint32_t ctotal = readlane(ci, 63);
        if (l == 0) { ms.sel_above_mass = total; ms.sel_need = ctotal; }
        if (bal != 0ull && l == __ffsll((long long)bal) - 1) {
            unsigned long long acc = wi - ws;
            uint32_t nacc = ci - cs;
            for (int j = 0; j < kMassBins / 64; ++j) {
                const int b = l * (kMassBins / 64) + j;
                if ((double)(acc + hw[b]) > target) {
                    ms.sel_digit = (uint32_t)b;
                    ms.hmass[0] = acc;          // mass above the bin
                    ms.sel_above_count = nacc;  // entries above the bin
                    ms.ib = (int)hn[b];         // entries in the bin
                    ms.flag = 1;
                    break;
                }
                acc += hw[b];
                nacc += hn[b];
            }
        }
    }
    __syncthreads();
    zk = ms.sel_above_mass;
    nk = (int)ms.sel_need;
    if (!ms.flag) { __syncthreads(); return 0; }
    const int bs = (int)ms.sel_digit, nb = ms.ib;
    const unsigned long long above = ms.hmass[0];
    const uint32_t above_count = ms.sel_above_count;
    __syncthreads();
    if (bs == kMassBins - 1 || nb > cap) return -1;
    // the bin's entries, sorted best first
    unsigned long long *G = reinterpret_cast<unsigned long long *>(raw);
    src.each([&](uint32_t, int idx, float y) {
        if (y > kNegInf && bin(y) == bs) {
            const int pos = wave_append(&ms.ncand);
            if (pos < cap) G[pos] = desc_key(y, idx);
        }
    });
    __syncthreads();
    const int n = min(ms.ncand, cap);
    sort_keys(G, n, ms.part);
    cut_in_sorted(G, n, above, above_count, (double)top_p * (double)zk, m, out, ms);
    return 1;
}

// Multi-pass row path: materialise the row's final scores in the workspace, then
// resolve top-k / top-p / the draw / top-N over the whole row.  Taken when the chunk
// candidates cannot settle the row.
template <typename TIn, int E>
__device__ __forceinline__ void dense_resolve(const Args &a, int row, const klsample_row_params &p, int mode,
                              unsigned char *raw, int *ids, Misc &ms) {
    constexpr int C = kThreads * E;
    const int V = a.V, S = a.S, tid = threadIdx.x;
    float *yb = a.ybuf + (size_t)row * a.ypitch;
    const bool pen = has_penalty(a, p, row);
    uint32_t *cnt = reinterpret_cast<uint32_t *>(raw);
    float mt = kNegInf;
    int at = 0x7fffffff;
    const TIn *src = reinterpret_cast<const TIn *>(a.logits) + (int64_t)row * a.row_stride;
    // Final scores into yb, chunk by chunk: E loads per thread (one per element, the
    // chunk's 256-element rows coalesced), the next chunk's requested before the current
    // one is penalised and written.  A history of at most kMaxChunksLds ids is kept in
    // LDS and counted from there per chunk; a longer one is re-read per chunk.
    int h0 = 0, h1 = 0;
    if (pen) hist_range(a, row, h0, h1);
    const int H = h1 - h0;
    const bool ids_lds = H <= kMaxChunksLds;
    if (pen && ids_lds) {
        for (int hb = 0; hb < H; hb += 8 * kThreads) {
            int id[8];
#pragma unroll
            for (int j = 0; j < 8; ++j) id[j] = a.hist_ids[h0 + min(hb + j * kThreads + tid, H - 1)];
#pragma unroll
            for (int j = 0; j < 8; ++j)
                if (hb + j * kThreads + tid < H) ids[hb + j * kThreads + tid] = id[j];
        }
    }
    const int spare = a.ypitch - 1;   // past every position a pass reads
    float xa[E], xb[E];
    auto request = [&](float (&x)[E], int c) {
        const int c0 = c * C, cn = min(C, V - c0);
#pragma unroll
        for (int j = 0; j < E; ++j) x[j] = Loader<TIn>::one(src + c0 + min(j * kThreads + tid, cn - 1));
    };
    request(xa, 0);
    for (int c = 0; c < S; ++c) {
        request(xb, min(c + 1, S - 1));
        const int c0 = c * C, cn = min(C, V - c0);
        if (pen) {
            uint4 *c4 = reinterpret_cast<uint4 *>(cnt);
            for (int i = tid; i < C / 4; i += kThreads) c4[i] = make_uint4(0u, 0u, 0u, 0u);
            __syncthreads();   // (also: the ids are in LDS)
            if (ids_lds) {
                for (int h = tid; h < H; h += kThreads) {
                    const unsigned rel = (unsigned)(ids[h] - c0);
                    if (rel < (unsigned)cn) atomicAdd(&cnt[rel], 1u);
                }
            } else {
                for (int hb = tid; hb < H; hb += 8 * kThreads) {
                    int id[8];
#pragma unroll
                    for (int j = 0; j < 8; ++j) id[j] = a.hist_ids[h0 + min(hb + j * kThreads, H - 1)];
#pragma unroll
                    for (int j = 0; j < 8; ++j) {
                        const unsigned rel = (unsigned)(id[j] - c0);
                        if (hb + j * kThreads < H && rel < (unsigned)cn) atomicAdd(&cnt[rel], 1u);
                    }
                }
            }
            __syncthreads();
        }
        // the counts first (one LDS wait), then the scores; every thread stores E values
        // (positions past the chunk go to the row's spare slot), so no branch separates
        // the stores from the loads in flight
        uint32_t kc[E];
#pragma unroll
        for (int j = 0; j < E; ++j) kc[j] = pen ? cnt[j * kThreads + tid] : 0u;
#pragma unroll
        for (int j = 0; j < E; ++j) {
            const int i = j * kThreads + tid;
            float y = xa[j];
            if (kc[j]) y = penalize(y, kc[j], p);
            if (mode != kGreedy) y = __fdiv_rn(y, p.temperature);
            const bool in = i < cn;
            yb[in ? c0 + i : spare] = y;
            if (in && y > mt) { mt = y; at = c0 + i; }
        }
#pragma unroll
        for (int j = 0; j < E; ++j) xa[j] = xb[j];
        if (pen) __syncthreads();   // the table is read before the next chunk clears it
    }
    const float m = block_max(mt, ms);
    int arg = block_min(mt == m ? at : 0x7fffffff, ms);
    if (arg == 0x7fffffff) arg = 0;
    __syncthreads();
    const double md = (double)m;
    auto wfix = [m](float y) -> unsigned long long { return weight_fix(y, m); };
    unsigned long long *sortbuf = reinterpret_cast<unsigned long long *>(raw);
    RowOut r;
    r.m = m;
    r.path = 1;
    const DenseSource all{yb, V, kNegInf, V};
    int count = 0;
    if (mode == kGreedy) {
        unsigned long long zq = 0ull;
        int nfin = 0;
        all.each([&](uint32_t, int, float y) { zq += wfix(y); nfin += (y > kNegInf) ? 1 : 0; });
        zq = block_sumq(zq, ms);
        nfin = block_sum(nfin, ms);
        r.token = arg;
        r.log_norm = log((double)zq / kFixScale);
        r.logprob = -r.log_norm;
        r.cut = kNegInf;
        r.cut_idx = V;
        r.kept = nfin;
        count = dense_topn(all, a.N, sortbuf, ms);
    } else {
        float lo = kNegInf;
        if (mode == kTopK) lo = fkey_inv(select_kth(all, (uint32_t)p.top_k, ms));
        const DenseSource ge{yb, V, lo, V};
        unsigned long long zk = 0ull;
        int nk = 0;
        float cut = lo;
        int cut_idx = V, kept = 0;
        unsigned long long zf = 0ull;
        int how = -1;   // top-p by mass bins: 1 cut, 0 nothing removed, -1 not settled
        if (p.flags & KLSAMPLE_ROW_TOP_P) {
            TopPCut tc;
            how = topp_cut_bins(ge, m, p.top_p, raw, 2 * kSortCap, zk, nk, tc, ms);
            if (how == 1) {
                cut = tc.cut;
                cut_idx = tc.cut_idx == 0x7fffffff ? V : tc.cut_idx;
                kept = tc.kept;
                zf = tc.zf;
            }
        } else {
            ge.each([&](uint32_t, int, float y) { zk += wfix(y); nk += (y > kNegInf) ? 1 : 0; });
            zk = block_sumq(zk, ms);
            nk = block_sum(nk, ms);
        }
        if (how != 1) {
            kept = nk;
            zf = zk;
        }
        if (how < 0 && (p.flags & KLSAMPLE_ROW_TOP_P)) {
            const double target = (double)p.top_p * (double)zk;
            MassPick mp;
            if (select_mass(ge, target, m, mp, ms)) {
                const unsigned long long wt = mp.group_count ? mp.group_mass / mp.group_count : 0ull;
                uint32_t keep = mp.group_count;
                if (wt > 0ull) {
                    const double room = target - (double)mp.above;
                    const double k = floor(room / (double)wt) + 1.0;
                    keep = (uint32_t)fmin((double)mp.group_count, fmax(1.0, k));
                }
                cut = fkey_inv(mp.key);
                kept = (int)(mp.above_count + keep);
                zf = mp.above + (unsigned long long)keep * wt;
                if (keep < mp.group_count) {
                    const float tie = cut;
                    int lastt;
                    double bt;
                    cut_idx = ordered_find(
                        V, [&](int i) { return yb[i] == tie ? 1.0 : 0.0; }, (double)keep - 0.5, ms, lastt, bt);
                    if (cut_idx < 0) cut_idx = V;
                }
            }
        }
        const DenseSource ks{yb, V, cut, cut_idx};
        int last;
        const unsigned long long tgt = (unsigned long long)floor((double)p.uniform * (double)zf);
        int tok = dense_draw(ks, m, tgt, ms, last);
        if (tok < 0) tok = last >= 0 ? last : 0;
        r.token = tok;
        r.cut = cut;
        r.cut_idx = cut_idx;
        r.kept = kept;
        r.log_norm = log((double)zf / kFixScale);
        r.logprob = (double)yb[tok] - md - r.log_norm;
        count = dense_topn(ks, a.N, sortbuf, ms);
    }
    write_row(a, row, mode, r, count, ms);
}

// A top-p row whose kept set reaches past the candidates; every chunk wrote its
// histogram and its final scores (wide_chunk).
//  1. The chunk histograms are merged into one over the row: chunk c's bin jc is row
//     bin jc + (G - G_c) (G of the row max m), its mass converted to units of 2^-40
//     relative to m (one rounding per chunk bin, identical wherever it is repeated).
//  2. The cut bin is the first whose running mass from the top exceeds p * total.
//  3. Per chunk: the mass of its bins above the cut bin.
//  4. One pass over the row's scores gathers the cut bin's entries, split 256 ways by
//     score; the crossing part, sorted, gives the crossing entry and the ties it keeps
//     (cut_in_sorted).
//  5. Each chunk's kept mass (step 3 and its kept cut-bin entries) gives the chunk where
//     the kept mass in vocab order crosses u * total; that chunk's scores are walked.
// `want` top-N entries are in ms.topn_*.  `ctab` holds kWideMaxChunks * 20 bytes and
// `raw` (kWideCross + kWideList) * 8 bytes of LDS.  Returns false, writing nothing, when
// the row cannot be resolved this way (cut in the last bin, a crossing part too large
// for LDS); dense_resolve runs.
constexpr int kWideList = 4096;    // cut-bin entries held in LDS
constexpr int kWideCross = 2048;   // entries of the crossing part of the cut bin

__device__ __forceinline__ bool wide_resolve(const Args &a, int row, const klsample_row_params &p, int mode, float m,
                                             int want, unsigned char *raw, unsigned long long *ctab, Misc &ms) {
    const int S = a.S, V = a.V, C = a.C, tid = threadIdx.x;
    const ChunkStat *st = a.stats + (size_t)row * S;
    const unsigned long long *hist = a.hist + (size_t)row * S * kWideBins;
    const float *yb = a.ybuf + (size_t)row * a.ypitch;
    uint32_t *hc = reinterpret_cast<uint32_t *>(raw);                                      // row bin counts
    unsigned long long *hm = reinterpret_cast<unsigned long long *>(raw + kWideBins * 4);  // row bin masses
    unsigned long long *D = reinterpret_cast<unsigned long long *>(raw);                   // crossing part (after 2)
    unsigned long long *L = reinterpret_cast<unsigned long long *>(raw + kWideCross * 8);  // cut-bin entries
    static_assert(kWideBins * 12 <= kWideCross * 8, "the row histogram fits below the list");
    unsigned long long *kc = ctab;                                           // per chunk: kept mass
    double *cf = reinterpret_cast<double *>(ctab + kWideMaxChunks);           // per chunk: mass conversion
    int *cd = reinterpret_cast<int *>(ctab + 2 * kWideMaxChunks);             // per chunk: bin offset G - G_c
    static_assert(2 * kWideMaxChunks * 8 + kWideMaxChunks * 4 <= kMaxChunksLds * 4,
                  "chunk tables fit the combine's count table");
    constexpr unsigned long long kMassMask = (1ull << kWideCountShift) - 1ull;
    constexpr double kUnit = (double)(1ull << (40 - kWideMassBits));
    const float G = floorf(m * kWideCells);
    for (int i = tid; i < kWideBins; i += kThreads) { hc[i] = 0u; hm[i] = 0ull; }
    for (int c = tid; c < S; c += kThreads) {
        const float Gc = floorf(st[c].m * kWideCells);
        cd[c] = (int)(G - Gc);
        cf[c] = exp((double)(Gc * (1.f / kWideCells)) - (double)m) * kUnit;
        kc[c] = 0ull;
    }
    __syncthreads();
    // chunk mass -> row units, rounded to the nearest integer (< 2^54): the two 32-bit
    // halves are converted separately (exact), cheaper than a 64-bit conversion
    auto conv = [&](unsigned long long v, int c) -> unsigned long long {
        const double x = rint((double)(v & kMassMask) * cf[c]);
        const double hi = floor(x * 2.3283064365386963e-10);   // x / 2^32
        const double lo = fma(hi, -4294967296.0, x);            // x - hi * 2^32, exact
        return ((unsigned long long)(uint32_t)hi << 32) | (uint32_t)lo;
    };
    // 1. merge: thread t reads words t, t + 256, ... of the row's chunk histograms
    //    (chunk c = word >> 10; each bin the difference of two prefix words), sixteen
    //    pairs of loads in flight
    static_assert(kWideBins == 1024, "chunk index = word >> 10");
    const int nw = S * kWideBins;
    for (int q0 = 0; q0 < nw; q0 += 16 * kThreads) {
        unsigned long long v[16], pv[16];
#pragma unroll
        for (int u = 0; u < 16; ++u) {
            const int q = min(q0 + u * kThreads + tid, nw - 1);
            v[u] = hist[q];
            pv[u] = hist[(q & (kWideBins - 1)) ? q - 1 : q];
        }
#pragma unroll
        for (int u = 0; u < 16; ++u) {
            const int q = q0 + u * kThreads + tid;
            const unsigned long long d = (q & (kWideBins - 1)) ? v[u] - pv[u] : v[u];
            if (q < nw && d != 0ull) {
                const int c = q >> 10, j = min((q & (kWideBins - 1)) + cd[c], kWideBins - 1);
                atomicAdd(&hc[j], (uint32_t)(d >> kWideCountShift));
                atomicAdd(&hm[j], conv(d, c));
            }
        }
    }
    __syncthreads();
    // 2. the cut bin: wave 0, 16 consecutive bins per lane
    if (wave_id() == 0) {
        const int l = lane_id();
        unsigned long long ws = 0ull;
        uint32_t cs = 0u;
#pragma unroll
        for (int j = 0; j < kWideBins / 64; ++j) { ws += hm[l * (kWideBins / 64) + j]; cs += hc[l * (kWideBins / 64) + j]; }
        const unsigned long long wi = wave_incl_scan(ws);
        const uint32_t ci = wave_incl_scan(cs);
        const unsigned long long total = readlane(wi, 63);
        const double target = (double)p.top_p * (double)total;
        const unsigned long long bal = __ballot((double)wi > target);
        if (l == 0) { ms.flag = 0; ms.da = target; }
        if (bal != 0ull && l == __ffsll((long long)bal) - 1) {
            unsigned long long acc = wi - ws;
            uint32_t nacc = ci - cs;
            for (int j = 0; j < kWideBins / 64; ++j) {
                const int b = l * (kWideBins / 64) + j;
                if ((double)(acc + hm[b]) > target) {
                    ms.sel_digit = (uint32_t)b;
                    ms.sel_above_mass = acc;
                    ms.sel_above_count = nacc;
                    ms.ib = (int)hc[b];
                    ms.flag = 1;
                    break;
                }
                acc += hm[b];
                nacc += hc[b];
            }
        }
    }
    __syncthreads();
    const int bstar = (int)ms.sel_digit, nb = ms.ib;
    const double target = ms.da;
    if (!ms.flag || bstar == kWideBins - 1 || nb < 1) return false;
    const unsigned long long above = ms.sel_above_mass;
    const uint32_t above_count = ms.sel_above_count;
    // 3. per chunk: the mass of its bins above the cut bin, one prefix word
    for (int c = tid; c < S; c += kThreads) {
        const int nc = min(kWideBins, bstar - cd[c]);
        kc[c] = nc > 0 ? conv(hist[(size_t)c * kWideBins + nc - 1], c) : 0ull;
    }
    if (tid == 0) ms.ncand = 0;
    for (int i = tid; i < 256; i += kThreads) { ms.hist[i] = 0u; ms.hmass[i] = 0ull; }
    __syncthreads();
    // 4. the cut bin's entries (scores in [lo_b, hi_b)): one pass over the row's scores,
    //    sixteen 16-byte loads per thread in flight, the next block requested before the
    //    current one is tested; split 256 ways by score (sub-bin 0 the highest; equal
    //    scores share one) and kept in L when the bin fits
    const float cell = G - (float)bstar;
    const float lo_b = cell * (1.f / kWideCells), hi_b = (cell + 1.f) * (1.f / kWideCells);
    const float sscale = 256.f * kWideCells;
    auto sub = [&](float y) { return min(255, (int)((hi_b - y) * sscale)); };
    const bool listed = nb <= kWideList;
    auto each_cut = [&](auto f) {   // f(score, index) over the cut bin's entries
        constexpr int U = 16;
        const int n4 = (V + 3) / 4;   // the buffer is readable up to V rounded up to 4
        const float4 *y4 = reinterpret_cast<const float4 *>(yb);
        float4 qa[U], qb[U];
        auto request = [&](float4 (&q)[U], int b0) {
#pragma unroll
            for (int u = 0; u < U; ++u) q[u] = y4[min(b0 + u * kThreads + tid, n4 - 1)];
        };
        request(qa, 0);
        for (int b0 = 0; b0 < n4; b0 += U * kThreads) {
            request(qb, b0 + U * kThreads);
#pragma unroll
            for (int u = 0; u < U; ++u) {
                const float t[4] = {qa[u].x, qa[u].y, qa[u].z, qa[u].w};
                bool any = false;
#pragma unroll
                for (int e = 0; e < 4; ++e) any |= (t[e] >= lo_b) & (t[e] < hi_b);
                if (any) {
                    const int i0 = 4 * (b0 + u * kThreads + tid);
#pragma unroll
                    for (int e = 0; e < 4; ++e)
                        if (t[e] >= lo_b && t[e] < hi_b && i0 + e < V && b0 + u * kThreads + tid < n4) f(t[e], i0 + e);
                }
            }
#pragma unroll
            for (int u = 0; u < U; ++u) qa[u] = qb[u];
        }
    };
    if (listed) {
        // The pass only lists the entries' indices: a lane marks its hits of a load
        // round in a 64-bit mask, and the wave reserves the round's list slots with one
        // atomic (the entries are sparse: anything done per entry inside the pass would
        // run with one or two lanes active and wait on LDS each time).  Their scores,
        // sub-bin counts and masses are then taken from the list with every lane busy.
        constexpr int U = 16;
        const int n4 = (V + 3) / 4;   // the buffer is readable up to V rounded up to 4
        const float4 *y4 = reinterpret_cast<const float4 *>(yb);
        float4 qa[U], qb[U];
        auto request = [&](float4 (&q)[U], int b0) {
#pragma unroll
            for (int u = 0; u < U; ++u) q[u] = y4[min(b0 + u * kThreads + tid, n4 - 1)];
        };
        request(qa, 0);
        for (int b0 = 0; b0 < n4; b0 += U * kThreads) {
            request(qb, b0 + U * kThreads);
            unsigned long long mask = 0ull;
#pragma unroll
            for (int u = 0; u < U; ++u) {
                const float t[4] = {qa[u].x, qa[u].y, qa[u].z, qa[u].w};
                const int vi = b0 + u * kThreads + tid;
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const bool hit = t[e] >= lo_b && t[e] < hi_b && 4 * vi + e < V && vi < n4;
                    mask |= (unsigned long long)hit << (4 * u + e);
                }
            }
            const uint32_t cnt = (uint32_t)__popcll(mask);
            const uint32_t incl = wave_incl_scan(cnt);
            const uint32_t total = readlane(incl, 63);
            if (total) {
                int base = 0;
                if (lane_id() == 0) base = atomicAdd(&ms.ncand, (int)total);
                int pos = __builtin_amdgcn_readfirstlane(base) + (int)(incl - cnt);
                while (mask) {
                    const int bit = __builtin_ctzll(mask);
                    mask &= mask - 1ull;
                    if (pos < kWideList) L[pos] = (unsigned long long)(4 * (b0 + (bit >> 2) * kThreads + tid) + (bit & 3));
                    ++pos;
                }
            }
#pragma unroll
            for (int u = 0; u < U; ++u) qa[u] = qb[u];
        }
        __syncthreads();
        const int nl = min(ms.ncand, kWideList);
        for (int i = tid; i < nl; i += kThreads) {
            const int idx = (int)L[i];
            const float y = yb[idx];
            L[i] = desc_key(y, idx);
            const int sb = sub(y);
            atomicAdd(&ms.hist[sb], 1u);
            atomicAdd(&ms.hmass[sb], weight_fix(y, m));
        }
    } else {
        each_cut([&](float y, int idx) {
            const int sb = sub(y);
            atomicAdd(&ms.hist[sb], 1u);
            atomicAdd(&ms.hmass[sb], weight_fix(y, m));
        });
    }
    __syncthreads();
    if (listed && ms.ncand != nb) return false;   // (the histogram and the scores always agree)
    if (wave_id() == 0) {
        const int l = lane_id();
        unsigned long long c[4], ws = 0ull;
        uint32_t n[4], ns = 0u;
#pragma unroll
        for (int j = 0; j < 4; ++j) { c[j] = ms.hmass[4 * l + j]; n[j] = ms.hist[4 * l + j]; ws += c[j]; ns += n[j]; }
        const unsigned long long wi = above + wave_incl_scan(ws);
        const uint32_t ni = above_count + wave_incl_scan(ns);
        const unsigned long long bal = __ballot((double)wi > target);
        // no sub-bin crossing (rounding): the last non-empty one is taken
        const unsigned long long nonempty = __ballot(ns > 0u);
        const int fl = bal ? __ffsll((long long)bal) - 1 : 63 - __clzll((long long)nonempty);
        if (l == fl) {
            // the lane's crossing sub-bin (or its last non-empty one), and the mass and
            // count above it (static indices only)
            unsigned long long acc = wi - ws, acc_at = acc;
            uint32_t nacc = ni - ns, nacc_at = nacc;
            int js = -1;
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const bool take = bal ? (js < 0 && (double)(acc + c[j]) > target) : (n[j] > 0u);
                if (take) { js = j; acc_at = acc; nacc_at = nacc; }
                acc += c[j];
                nacc += n[j];
            }
            ms.sel_need = (uint32_t)(4 * l + max(js, 0));
            ms.sel_above_mass = acc_at;
            ms.sel_above_count = nacc_at;
        }
        if (l == 0) ms.ncand = 0;
    }
    __syncthreads();
    const int sstar = (int)ms.sel_need;
    const unsigned long long above_s = ms.sel_above_mass;
    const uint32_t above_count_s = ms.sel_above_count;
    if (listed) {
        for (int i = tid; i < nb; i += kThreads) {
            const unsigned long long k = L[i];
            if (sub(desc_key_y(k)) == sstar) {
                const int pos = wave_append(&ms.ncand);
                if (pos < kWideCross) D[pos] = k;
            }
        }
    } else {
        // a bin larger than the list: the crossing sub-bin from a second pass
        each_cut([&](float y, int idx) {
            if (sub(y) == sstar) {
                const int pos = wave_append(&ms.ncand);
                if (pos < kWideCross) D[pos] = desc_key(y, idx);
            }
        });
    }
    __syncthreads();
    const int ns = ms.ncand;
    if (ns > kWideCross) return false;
    sort_keys(D, ns, ms.part);
    TopPCut tc;
    cut_in_sorted(D, ns, above_s, above_count_s, target, m, tc, ms);
    const float cut = tc.cut;
    const int cut_idx = tc.cut_idx == 0x7fffffff ? V : tc.cut_idx;
    const unsigned long long zf = tc.zf;
    auto kept = [&](float y, int idx) { return y > cut || (y == cut && idx <= cut_idx); };
    // 5. each chunk's kept cut-bin entries (a third pass over the scores when they were
    //    not listed)
    if (listed) {
        for (int i = tid; i < nb; i += kThreads) {
            const float y = desc_key_y(L[i]);
            const int idx = desc_key_idx(L[i]);
            if (kept(y, idx)) atomicAdd(&kc[idx / C], weight_fix(y, m));
        }
    } else {
        each_cut([&](float y, int idx) {
            if (kept(y, idx)) atomicAdd(&kc[idx / C], weight_fix(y, m));
        });
    }
    __syncthreads();
    // the chunk where the kept mass in vocab order crosses u * total
    const unsigned long long tgt = (unsigned long long)floor((double)p.uniform * (double)zf);
    if (wave_id() == 0) {
        const int l = lane_id();
        unsigned long long run = 0ull, before = 0ull;
        int cs = -1, clast = -1;
        for (int c0 = 0; c0 < S && cs < 0; c0 += 64) {
            const int c = c0 + l;
            const unsigned long long w = c < S ? kc[c] : 0ull;
            const unsigned long long incl = run + wave_incl_scan(w);
            const unsigned long long bal = __ballot(c < S && incl > tgt);
            const unsigned long long pos = __ballot(w > 0ull);
            if (pos) clast = c0 + 63 - __clzll((long long)pos);
            if (bal) {
                const int fl = __ffsll((long long)bal) - 1;
                cs = c0 + fl;
                before = readlane(incl - w, fl);
            }
            run = readlane(incl, 63);
        }
        if (cs < 0) { cs = clast >= 0 ? clast : 0; before = 0ull; }   // (rounding)
        if (l == 0) { ms.ia = cs; ms.sel_above_mass = before; }
    }
    __syncthreads();
    const int cs = ms.ia;
    const unsigned long long rem = tgt - min(tgt, ms.sel_above_mass);
    __syncthreads();
    // its scores walked in vocab order (the last kept one if rounding leaves it short)
    const int c0 = cs * C, cn = min(C, V - c0);
    const DenseSource ks{yb + c0, cn, cut, cut_idx - c0};
    int last;
    int tok = dense_draw(ks, m, rem, ms, last);
    if (tok < 0) tok = last >= 0 ? last : 0;
    RowOut r;
    r.token = c0 + tok;
    r.m = m;
    r.cut = cut;
    r.cut_idx = cut_idx;
    r.kept = tc.kept;
    r.log_norm = log((double)zf / kFixScale);
    r.logprob = (double)yb[r.token] - (double)m - r.log_norm;
    r.path = 2;
    write_row(a, row, mode, r, min(want, tc.kept), ms);
    return true;
}

// The kept entries of an LDS list of sort keys (for radix selects).
struct KeptListSource {
    const unsigned long long *E;
    int n;
    float cut;
    int cut_idx;
    template <class F>
    __device__ __forceinline__ void each(F f) const {
        for (int i = threadIdx.x; i < n; i += kThreads) {
            const unsigned long long k = E[i];
            const float y = desc_key_y(k);
            const int idx = desc_key_idx(k);
            if (y > cut || (y == cut && idx <= cut_idx)) f(fkey(y), idx, y);
        }
    }
};

// Finish a sampled row from the unsorted list E[0..n) of sort keys (final-space scores),
// which holds every entry of the row scoring at least its smallest score.  Nothing of
// size n is sorted: each step is a 256-way histogram over the list and a sort of the
// crossing part only.
//  * top-p (`topp`): the cut in exclusive form against p * Z, Z = `zrow` (units of 2^-40
//    relative to the list's max; the whole row's mass for top-p-only rows) or, for
//    zrow < 0, the list's own mass (top-k rows);
//  * the draw: the kept mass in vocab order, over 256 index ranges, then the crossing
//    range sorted by index and walked;
//  * top-N: a radix select of the N-th kept score, the kept entries reaching it sorted.
// `W` is LDS for kSortCap keys, apart from E.  Returns false, writing nothing, when the
// top-p cut does not fall within E and E is not the whole row (`complete`).
__device__ __forceinline__ bool finish_list(const Args &a, int row, int mode, const klsample_row_params &p,
                                            const unsigned long long *E, int n, bool topp, double zrow,
                                            bool complete, unsigned long long *W, Misc &ms) {
    const int V = a.V, N = a.N, tid = threadIdx.x;
    uint32_t kmin = 0xffffffffu, kmax = 0u;
    for (int i = tid; i < n; i += kThreads) {
        const uint32_t k = fkey(desc_key_y(E[i]));
        kmin = min(kmin, k);
        kmax = max(kmax, k);
    }
    kmin = block_reduce(kmin, OpMinU(), ms.red.u, 0xffffffffu);
    kmax = block_reduce(kmax, OpMaxU(), ms.red.u, 0u);
    const float ylo = fkey_inv(kmin), yhi = fkey_inv(kmax);
    const float mref = yhi;
    TopPCut tc;
    tc.cut = kNegInf;
    tc.cut_idx = 0x7fffffff;
    tc.kept = n;
    tc.zf = 0ull;
    bool cut_all = true;   // every entry kept
    if (topp || zrow < 0.0) {
        unsigned long long z = 0ull;
        for (int i = tid; i < n; i += kThreads) z += weight_fix(desc_key_y(E[i]), mref);
        tc.zf = block_sumq(z, ms);
    }
    if (topp) {
        // 256 score bins over [ylo, yhi], bin 0 the highest (equal scores share a bin)
        const float span = yhi - ylo;
        float scale = span > 0.f ? 256.f / span : 0.f;
        if (!(scale <= __FLT_MAX__)) scale = 0.f;
        auto bin = [&](float y) { return min(255, (int)((yhi - y) * scale)); };
        for (int i = tid; i < 256; i += kThreads) { ms.hist[i] = 0u; ms.hmass[i] = 0ull; }
        __syncthreads();
        for (int i = tid; i < n; i += kThreads) {
            const float y = desc_key_y(E[i]);
            atomicAdd(&ms.hist[bin(y)], 1u);
            atomicAdd(&ms.hmass[bin(y)], weight_fix(y, mref));
        }
        __syncthreads();
        const double target = (double)p.top_p * (zrow >= 0.0 ? zrow : (double)tc.zf);
        if (wave_id() == 0) {
            const int l = lane_id();
            unsigned long long c[4], ws = 0ull;
            uint32_t nn[4], ns = 0u;
#pragma unroll
            for (int j = 0; j < 4; ++j) { c[j] = ms.hmass[4 * l + j]; nn[j] = ms.hist[4 * l + j]; ws += c[j]; ns += nn[j]; }
            const unsigned long long wi = wave_incl_scan(ws);
            const uint32_t ni = wave_incl_scan(ns);
            const unsigned long long bal = __ballot((double)wi > target);
            if (l == 0) ms.flag = bal ? 1 : 0;
            if (bal && l == __ffsll((long long)bal) - 1) {
                unsigned long long acc = wi - ws, acc_at = acc;
                uint32_t nacc = ni - ns, nacc_at = nacc;
                int js = -1;
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    if (js < 0 && (double)(acc + c[j]) > target) { js = j; acc_at = acc; nacc_at = nacc; }
                    acc += c[j];
                    nacc += nn[j];
                }
                ms.sel_need = (uint32_t)(4 * l + max(js, 0));
                ms.sel_above_mass = acc_at;
                ms.sel_above_count = nacc_at;
            }
            if (l == 0) ms.ncand = 0;
        }
        __syncthreads();
        if (ms.flag) {
            // the crossing bin, sorted, gives the crossing entry and the ties it keeps
            const int bs = (int)ms.sel_need;
            const unsigned long long above = ms.sel_above_mass;
            const uint32_t above_count = ms.sel_above_count;
            for (int i = tid; i < n; i += kThreads) {
                const unsigned long long k = E[i];
                if (bin(desc_key_y(k)) == bs) W[wave_append(&ms.ncand)] = k;
            }
            __syncthreads();
            const int nb = ms.ncand;
            sort_keys(W, nb, ms.part);
            cut_in_sorted(W, nb, above, above_count, target, mref, tc, ms);
            cut_all = false;
        } else if (!complete) {
            return false;   // the kept mass reaches past the list
        }
    }
    // (nothing cut: the list's smallest score, every entry scoring it being listed)
    const float cut = cut_all ? ylo : tc.cut;
    const int cut_idx = (cut_all || tc.cut_idx == 0x7fffffff) ? V : tc.cut_idx;
    const int kept_n = cut_all ? n : tc.kept;
    const unsigned long long zf = tc.zf;
    auto kept = [&](float y, int idx) { return y > cut || (y == cut && idx <= cut_idx); };
    // the draw: kept mass over 256 index ranges, then the crossing range sorted by index
    const int rw = (V + 255) / 256;
    for (int i = tid; i < 256; i += kThreads) { ms.hist[i] = 0u; ms.hmass[i] = 0ull; }
    __syncthreads();
    for (int i = tid; i < n; i += kThreads) {
        const float y = desc_key_y(E[i]);
        const int idx = desc_key_idx(E[i]);
        if (kept(y, idx)) {
            atomicAdd(&ms.hist[idx / rw], 1u);
            atomicAdd(&ms.hmass[idx / rw], weight_fix(y, mref));
        }
    }
    __syncthreads();
    const unsigned long long tgt = (unsigned long long)floor((double)p.uniform * (double)zf);
    if (wave_id() == 0) {
        const int l = lane_id();
        unsigned long long c[4], ws = 0ull;
        uint32_t nn[4], ns = 0u;
#pragma unroll
        for (int j = 0; j < 4; ++j) { c[j] = ms.hmass[4 * l + j]; nn[j] = ms.hist[4 * l + j]; ws += c[j]; ns += nn[j]; }
        const unsigned long long wi = wave_incl_scan(ws);
        const unsigned long long bal = __ballot(wi > tgt);
        const unsigned long long nonempty = __ballot(ns > 0u);
        // (no range crossing: rounding; the last kept entry is taken)
        const int fl = bal ? __ffsll((long long)bal) - 1 : 63 - __clzll((long long)nonempty);
        if (l == fl) {
            unsigned long long acc = wi - ws, acc_at = acc;
            int js = -1;
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const bool take = bal ? (js < 0 && acc + c[j] > tgt) : (nn[j] > 0u);
                if (take) { js = j; acc_at = acc; }
                acc += c[j];
            }
            ms.ib = 4 * l + max(js, 0);
            ms.sel_above_mass = bal ? acc_at : ~0ull;
        }
        if (l == 0) ms.ncand = 0;
    }
    __syncthreads();
    const int rr = ms.ib;
    const unsigned long long rem = ms.sel_above_mass == ~0ull ? ~0ull : tgt - ms.sel_above_mass;
    for (int i = tid; i < n; i += kThreads) {
        const float y = desc_key_y(E[i]);
        const int idx = desc_key_idx(E[i]);
        if (kept(y, idx) && idx / rw == rr)
            W[wave_append(&ms.ncand)] = ((unsigned long long)(uint32_t)idx << 32) | __float_as_uint(y);
    }
    __syncthreads();
    const int nr = ms.ncand;
    sort_keys(W, nr, ms.part);
    if (wave_id() == 0) {
        const int l = lane_id();
        unsigned long long run = 0ull;
        int found = -1;
        for (int i0 = 0; i0 < nr && found < 0; i0 += 64) {
            const int i = i0 + l;
            const unsigned long long w = i < nr ? weight_fix(__uint_as_float((uint32_t)W[i]), mref) : 0ull;
            const unsigned long long incl = run + wave_incl_scan(w);
            const unsigned long long bal = __ballot(i < nr && incl > rem);
            if (bal) found = i0 + __ffsll((long long)bal) - 1;
            run = readlane(incl, 63);
        }
        if (found < 0) found = max(nr - 1, 0);
        if (l == 0) ms.ia = found;
    }
    __syncthreads();
    const unsigned long long kt = W[ms.ia];
    RowOut r;
    r.token = (int)(kt >> 32);
    r.m = mref;
    r.cut = cut;
    r.cut_idx = cut_idx;
    r.kept = kept_n;
    r.log_norm = log((double)zf / kFixScale);
    r.logprob = (double)__uint_as_float((uint32_t)kt) - (double)mref - r.log_norm;
    r.path = 0;
    // top-N: the N-th kept score by radix select, the kept entries reaching it sorted
    const int want = min(N, kept_n);
    __syncthreads();   // (W is read before it is reused)
    if (want > 0) {
        const KeptListSource ks{E, n, cut, cut_idx};
        const uint32_t kn = select_kth(ks, (uint32_t)want, ms);
        if (tid == 0) ms.ncand = 0;
        __syncthreads();
        ks.each([&](uint32_t key, int idx, float y) {
            if (key >= kn) {
                const int pos = wave_append(&ms.ncand);
                if (pos < kSortCap) W[pos] = desc_key(y, idx);
            }
        });
        __syncthreads();
        const int t = min(ms.ncand, kSortCap);
        sort_keys(W, t, ms.part);
        for (int i = tid; i < want; i += kThreads) {
            ms.topn_idx[i] = desc_key_idx(W[i]);
            ms.topn_y[i] = desc_key_y(W[i]);
        }
        __syncthreads();
    }
    write_row(a, row, mode, r, want, ms);
    return true;
}

// Resolve one row from its chunk summaries and candidates (or hand it to
// dense_resolve).  Runs in one workgroup of kThreads.
// Copy the entries of `src` scoring >= lo into the LDS list `dst` (capacity cap);
// returns how many there were (the list holds min(count, cap) of them).
template <typename Src>
__device__ __forceinline__ int gather_keys(const Src &src, float lo, unsigned long long *dst, int cap, Misc &ms) {
    if (threadIdx.x == 0) ms.ncand = 0;
    __syncthreads();
    src.each([&](uint32_t, int idx, float y) {
        if (y >= lo) {
            const int pos = wave_append(&ms.ncand);
            if (pos < cap) dst[pos] = desc_key(y, idx);
        }
    });
    __syncthreads();
    return ms.ncand;
}

// ---------------------------------------------------------------------------------
// One-wave finish of a row whose kept set is small: no barriers, one key per lane.

// Sort D[0..n) ascending (best first) in LDS with the whole block.
__device__ __forceinline__ void sort_top(unsigned long long *D, int n, Misc &ms) {
    sort_keys(D, n, ms.part);
}

// Kept prefix of D[0..n) (sorted best first, n <= 64) under top-p: the first entry whose
// exclusive mass exceeds p * zref is the last one kept.  Returns its count, or -1 if no
// entry of D crosses.  Wave-uniform; call from one whole wave.
__device__ __forceinline__ int wave_topp(const unsigned long long *D, int n, double mref, double zref, float top_p) {
    const int l = lane_id();
    const double w = l < n ? (double)__expf(desc_key_y(D[l]) - (float)mref) : 0.0;
    const double excl = wave_shift_excl(wave_incl_scan(w));
    const unsigned long long cross = __ballot(l < n && excl > (double)top_p * zref);
    return cross ? __ffsll((long long)cross) - 1 : -1;
}

// Row outputs from one wave: token, logprob, row state, and the top-N list taken from
// D[0..count) (best first); count <= 64 and N <= 64.  Same contents as write_row.
__device__ __forceinline__ void wave_write(const Args &a, int row, int mode, const RowOut &r,
                                           const unsigned long long *D, int count) {
    const int N = a.N, V = a.V;
    const int l = lane_id();
    if (N > 0) {
        const int nv = min(N, V);
        int32_t *ids = a.top_ids + (size_t)row * N;
        float *lps = a.top_lp + (size_t)row * N;
        const int idx = l < count ? desc_key_idx(D[l]) : -1;
        if (l < count && l < nv) {
            ids[l] = idx;
            lps[l] = (float)((double)desc_key_y(D[l]) - (double)r.m - r.log_norm);
        } else if (l >= nv && l < N) {
            ids[l] = -1;
            lps[l] = kNegInf;
        }
        if (count < nv) {
            // fillers: the smallest ids not listed, all below 128 since count, nv <= 64
            bool hit_lo = false, hit_hi = false;
            for (int j = 0; j < count; ++j) {
                const int ij = __builtin_amdgcn_readlane(idx, j);
                hit_lo |= (ij == l);
                hit_hi |= (ij == l + 64);
            }
            const unsigned long long free_lo = ~__ballot(hit_lo), free_hi = ~__ballot(hit_hi);
            const unsigned long long below = (1ull << l) - 1ull;
            const int need = nv - count;
            const int r_lo = __popcll(free_lo & below);
            if (((free_lo >> l) & 1ull) && r_lo < need) {
                ids[count + r_lo] = l;
                lps[count + r_lo] = kNegInf;
            }
            const int r_hi = __popcll(free_lo) + __popcll(free_hi & below);
            if (((free_hi >> l) & 1ull) && r_hi < need) {
                ids[count + r_hi] = l + 64;
                lps[count + r_hi] = kNegInf;
            }
        }
    }
    if (l == 0) {
        a.token[row] = r.token;
        append_token(a, row, r.token);
        a.logprob[row] = (float)r.logprob;
        klsample_row_info info;
        info.max_score = r.m;
        info.cut_score = r.cut;
        info.cut_index = r.cut_idx;
        info.kept = r.kept;
        info.log_norm = r.log_norm;
        info.path = r.path;
        info.mode = mode;
        a.rows[row] = info;
        if (a.row_info) a.row_info[row] = info;
    }
}

// Finish a sampled row in one wave: D[0..n) sorted best first, the first L kept
// (1 <= L <= 64, L <= n), N <= 64; `scr` is 128 free LDS words of 8 bytes.  Same
// results as finish_list.  The draw ranks the kept entries by vocab index (broadcast
// LDS reads, or `irank`), places their weights in index order and takes one prefix scan.
// `wz`, when given, holds the lane's weight exp(y - mref) and the kept entries' sum.
__device__ __forceinline__ void wave_finish(const Args &a, int row, int mode, const klsample_row_params &p,
                                            const unsigned long long *D, int n, int L, double mref,
                                            unsigned long long *scr, const uint32_t *irank = nullptr,
                                            bool ranked_all = false, const double *wz = nullptr) {
    const int l = lane_id();
    const bool kept = l < L;
    // ranked_all: irank holds vocab-order ranks among all n <= 64 entries; the entries
    // past the kept prefix then take part in the ordered draw with weight 0
    const bool placed = ranked_all ? (l < n) : kept;
    const unsigned long long key = placed ? D[l] : ~0ull;
    const float y = placed ? desc_key_y(key) : kNegInf;
    const int idx = placed ? desc_key_idx(key) : 0x7fffffff;
    // wz (optional): the lane's weight and the kept sum, already computed by the caller
    const double w = wz ? (kept ? wz[0] : 0.0) : (kept ? (double)__expf(y - (float)mref) : 0.0);
    int rank = 0;
    if (irank != nullptr) {
        rank = placed ? (int)irank[l] : 0;
    } else {
#pragma unroll 4
        for (int j = 0; j < L; j += 2) {
            const ulonglong2 q = *reinterpret_cast<const ulonglong2 *>(&D[j]);
            rank += (desc_key_idx(q.x) < idx) ? 1 : 0;
            rank += (j + 1 < L && desc_key_idx(q.y) < idx) ? 1 : 0;
        }
    }
    const double zf = wz ? wz[1] : wave_reduce(w, OpSumD(), 0.0);
    RowOut r;
    r.path = 0;
    r.m = (float)mref;
    r.cut = readlane(y, L - 1);
    r.cut_idx = (L < n && desc_key_y(D[L]) == r.cut) ? __builtin_amdgcn_readlane(idx, L - 1) : a.V;
    r.kept = L;
    r.log_norm = (double)logf((float)zf);   // zf >= 1: float accuracy (~1e-7 absolute) suffices
    __builtin_amdgcn_wave_barrier();
    if (placed) {
        scr[rank] = __double_as_longlong(w);
        scr[64 + rank] = (unsigned long long)(uint32_t)idx | (kept ? (1ull << 32) : 0ull);
    }
    __builtin_amdgcn_wave_barrier();
    // lane i now holds the i-th smallest placed index: inverse CDF in vocab order
    const bool at_placed = ranked_all ? (l < n) : kept;
    const unsigned long long sv = at_placed ? scr[64 + l] : 0ull;
    const bool kf = (sv >> 32) != 0ull;
    const double wi = at_placed ? __longlong_as_double(scr[l]) : 0.0;
    const int ii = (int)(uint32_t)sv;
    const double cum = wave_incl_scan(wi);
    const double target = (double)p.uniform * zf;
    const unsigned long long over = __ballot(kf && cum > target);
    int lt;
    if (over) {
        lt = __ffsll((long long)over) - 1;
    } else {
        const unsigned long long pos = __ballot(kf && wi > 0.0);
        lt = pos ? 63 - __clzll((long long)pos) : 0;
    }
    r.token = __builtin_amdgcn_readlane(ii, lt);
    const unsigned long long at = __ballot(kept && idx == r.token);
    const int lo = at ? __ffsll((long long)at) - 1 : 0;
    r.logprob = (double)readlane(y, lo) - mref - r.log_norm;
    wave_write(a, row, mode, r, D, min(a.N, L));
}

// Copy the entries of A[0..n) scoring >= t into D (capacity cap); returns their count
// (D holds min(count, cap) of them).  Entries are counted first and one LDS atomic per
// wave reserves their places.
__device__ __forceinline__ int gather_ge(const unsigned long long *A, int n, float t, unsigned long long *D, int cap,
                                         Misc &ms) {
    if (threadIdx.x == 0) ms.ncand = 0;
    __syncthreads();
    int mine = 0;
    for (int i = threadIdx.x; i < n; i += kThreads) mine += (desc_key_y(A[i]) >= t) ? 1 : 0;
    const int incl = wave_incl_scan(mine);
    int base = 0;
    if (lane_id() == 63 && incl > 0) base = atomicAdd(&ms.ncand, incl);
    base = readlane(base, 63) + incl - mine;
    for (int i = threadIdx.x; i < n; i += kThreads) {
        const unsigned long long k = A[i];
        if (desc_key_y(k) >= t) {
            if (base < cap) D[base] = k;
            ++base;
        }
    }
    __syncthreads();
    return ms.ncand;
}

// ---------------------------------------------------------------------------------
// The R best of A[0..n) (n > R >= 1) and every entry tied with the R-th, sorted best
// first into D[0..cap).  Returns their count, or -1 if they do not fit.  One linear
// 256-bin histogram over the entries' range [ylo, yhi] usually isolates them (the
// bins above the R-th entry's bin, plus that bin); otherwise an exact radix select.
__device__ __forceinline__ int select_top(const unsigned long long *A, int n, int R, float ylo, float yhi,
                                          unsigned long long *D, int cap, Misc &ms) {
    const double span = (double)yhi - (double)ylo;
    int t = cap + 1;
    if (span > 0.0) {
        const double scale = 256.0 / span;
        auto bin = [&](unsigned long long k) {
            return min(255, (int)(((double)desc_key_y(k) - (double)ylo) * scale));
        };
        for (int i = threadIdx.x; i < 256; i += kThreads) ms.hist[i] = 0u;
        __syncthreads();
        for (int i = threadIdx.x; i < n; i += kThreads) atomicAdd(&ms.hist[bin(A[i])], 1u);
        __syncthreads();
        pick_digit_count(ms, (uint32_t)R);
        const int b = (int)ms.sel_digit;
        __syncthreads();
        if (threadIdx.x == 0) ms.ncand = 0;
        __syncthreads();
        int mine = 0;
        for (int i = threadIdx.x; i < n; i += kThreads) mine += (bin(A[i]) >= b) ? 1 : 0;
        const int incl = wave_incl_scan(mine);
        int base = 0;
        if (lane_id() == 63 && incl > 0) base = atomicAdd(&ms.ncand, incl);
        base = readlane(base, 63) + incl - mine;
        for (int i = threadIdx.x; i < n; i += kThreads) {
            const unsigned long long k = A[i];
            if (bin(k) >= b) {
                if (base < cap) D[base] = k;
                ++base;
            }
        }
        __syncthreads();
        t = ms.ncand;
    }
    if (t > cap) {
        // the R-th entry's bin is crowded (or every entry is equal): exact radix select
        const LdsSource src{A, n};
        const float tau = fkey_inv(select_kth(src, (uint32_t)R, ms));
        t = gather_keys(src, tau, D, cap, ms);
        if (t > cap) return -1;
    }
    sort_top(D, t, ms);
    // keep the R best and the ties of the R-th
    const float tau = desc_key_y(D[R - 1]);
    int c = 0;
    for (int i = R + (int)threadIdx.x; i < t; i += kThreads) c += (desc_key_y(D[i]) == tau) ? 1 : 0;
    return R + block_sum(c, ms);
}

// Smallest float x with fl(x / T) >= y (T > 0): fl(x / T) is non-decreasing in x, so
// {x : fl(x / T) >= y} = {x : x >= that value}.  Found by stepping from fl(y * T), whose
// distance from it is a few ulps; +inf when no finite x qualifies, -inf for y = -inf.
__device__ __forceinline__ float quotient_threshold(float y, float T) {
    if (!(y > kNegInf)) return kNegInf;
    if (T == 1.f) return y;   // fl(x / 1) = x
    float x = __fmul_rn(y, T);
    if (!(fabsf(x) <= __FLT_MAX__)) x = x > 0.f ? __FLT_MAX__ : -__FLT_MAX__;
    for (int i = 0; i < 64 && !(__fdiv_rn(x, T) >= y); ++i) {
        if (x == __FLT_MAX__) return __builtin_huge_valf();
        x = nextafterf(x, __builtin_huge_valf());
    }
    for (int i = 0; i < 64; ++i) {
        const float xp = nextafterf(x, kNegInf);
        if (!(__fdiv_rn(xp, T) >= y)) break;
        x = xp;
    }
    return x;
}

// Block: the entries of A[0..n) (n > R >= 1) in the linear histogram bins (256 over
// [ylo, yhi]) at or above the bin of the R-th largest, into D (capacity cap), unsorted.
// ms.hist must be zero unless ms_hist_dirty (then it is cleared first) and ms.ib the
// zero counter.  Returns their count (D holds at most cap of them), or -1 for a
// degenerate range.  Two barriers: every wave finds the bin from the same histogram.
__device__ __forceinline__ int hist_gather(const unsigned long long *A, int n, int R, float ylo, float yhi,
                                           unsigned long long *D, int cap, Misc &ms, bool ms_hist_dirty) {
    const float span = yhi - ylo;
    const float scale = 256.f / span;
    if (!(span > 0.f) || !(scale <= __FLT_MAX__)) return -1;
    auto bin = [&](unsigned long long k) { return min(255, (int)((desc_key_y(k) - ylo) * scale)); };
    if (ms_hist_dirty) {
        for (int i = threadIdx.x; i < 256; i += kThreads) ms.hist[i] = 0u;
        __syncthreads();
    }
    // each thread's entries (n <= kSortCap: at most kPer) and their bins stay in
    // registers between the two passes
    constexpr int kPer = kSortCap / kThreads;
    unsigned long long key[kPer];
    int bn[kPer];
#pragma unroll
    for (int j = 0; j < kPer; ++j) {
        const int i = threadIdx.x + j * kThreads;
        key[j] = A[min(i, n - 1)];
        bn[j] = (i < n) ? bin(key[j]) : -1;
    }
    // rounds past n are skipped by the whole block; in the last one, lanes past n add 0
    // (no per-entry branch)
#pragma unroll
    for (int j = 0; j < kPer; ++j) {
        if (j * kThreads >= n) break;
        atomicAdd(&ms.hist[max(bn[j], 0)], bn[j] >= 0 ? 1u : 0u);
    }
    __syncthreads();
    const int l = lane_id();
    uint32_t c[4], sum = 0u;
#pragma unroll
    for (int j = 0; j < 4; ++j) { c[j] = ms.hist[255 - 4 * l - j]; sum += c[j]; }
    const uint32_t incl = wave_incl_scan(sum);
    const unsigned long long reach = __ballot(incl >= (uint32_t)R);
    const int fl = reach ? __ffsll((long long)reach) - 1 : 63;
    int b = 0;
    if (l == fl) {
        uint32_t acc = incl - sum;
        b = 252 - 4 * l;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            if (acc + c[j] >= (uint32_t)R) { b = 255 - 4 * l - j; break; }
            acc += c[j];
        }
    }
    b = __builtin_amdgcn_readlane(b, fl);
    int mine = 0;
#pragma unroll
    for (int j = 0; j < kPer; ++j) mine += (bn[j] >= b) ? 1 : 0;
    const int pincl = wave_incl_scan(mine);
    int base = 0;
    if (l == 63 && pincl > 0) base = atomicAdd(&ms.ib, pincl);
    base = readlane(base, 63) + pincl - mine;
    unsigned long long *const sink = &ms.sink[threadIdx.x];
#pragma unroll
    for (int j = 0; j < kPer; ++j) {   // branch-free: the others go to the thread's sink
        if (j * kThreads >= n) break;
        const bool ok = bn[j] >= b;
        *((ok && base < cap) ? &D[base] : sink) = key[j];
        base += ok ? 1 : 0;
    }
    __syncthreads();
    return ms.ib;
}


// Emit a row's outputs with its top-N list in D[0..count): one wave when the list is
// short, else the block writer.
__device__ __forceinline__ void emit_row(const Args &a, int row, int mode, const RowOut &r,
                                         const unsigned long long *D, int count, Misc &ms) {
    if (count <= 64 && a.N <= 64) {
        if (wave_id() == 0) wave_write(a, row, mode, r, D, count);
        return;
    }
    for (int t = threadIdx.x; t < count; t += kThreads) {
        ms.topn_idx[t] = desc_key_idx(D[t]);
        ms.topn_y[t] = desc_key_y(D[t]);
    }
    __syncthreads();
    write_row(a, row, mode, r, count, ms);
}

constexpr int kTopPShort = 48;   // top-p rows first try a kept set within their best 48
constexpr int kSpecLoads = 8;    // candidate pairs each thread requests with the chunk summaries
constexpr int kSpecPairs = 64;   // ... out of the first pairs of each chunk

// The first memory requests of a row's combine: its chunk summaries and the first
// candidate pairs of its first chunks, in one round trip, issued before the row's
// parameters are read (they depend on nothing but the launch).  Greedy and full rows
// without top-N read slots they ignore.
struct RowSpec {
    uint4 spec[kSpecLoads];
    ChunkStat s0;   // the summary of chunk threadIdx.x (clamped)
};

__device__ __forceinline__ void spec_layout(const Args &a, int &ppc, int &pshift, int &nspec) {
    ppc = min(a.cand_cap / 2, kSpecPairs);   // a power of two
    pshift = 31 - __clz(ppc);
    nspec = min(a.S, (kSpecLoads * kThreads) >> pshift);
}

// A row's parameters, loaded by every lane from the same address through the vector
// memory path and made wave-uniform again.  (A scalar load would be waited for together
// with any other scalar load, e.g. of a kernel argument, issued after it.)
__device__ __forceinline__ klsample_row_params load_params_vmem(const klsample_row_params *P, int row) {
    int z;
    __asm__ volatile("v_mov_b32 %0, 0" : "=v"(z));   // a lane-varying zero: keeps the load a vector load
    const uint32_t *q = reinterpret_cast<const uint32_t *>(P + row) + z;   // 4-byte aligned
    uint32_t w[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) w[i] = q[i];
    klsample_row_params p;
    static_assert(sizeof(p) == sizeof(w), "row parameters are 32 bytes");
#pragma unroll
    for (int i = 0; i < 8; ++i) w[i] = __builtin_amdgcn_readfirstlane(w[i]);
    __builtin_memcpy(&p, w, sizeof(p));
    return p;
}

__device__ __forceinline__ void request_row(const Args &a, int row, RowSpec &r) {
    int ppc, pshift, nspec;
    spec_layout(a, ppc, pshift, nspec);
    const Cand *rc = a.cands + (size_t)row * a.S * a.cand_cap;
    // (addresses are clamped into range rather than the loads predicated: a predicated
    // load would be waited for before the next one is issued)
#pragma unroll
    for (int i = 0; i < kSpecLoads; ++i) {
        const int q = threadIdx.x + i * kThreads;
        const int c = min(q >> pshift, max(nspec - 1, 0));
        r.spec[i] = reinterpret_cast<const uint4 *>(rc + (size_t)c * a.cand_cap)[q & (ppc - 1)];
    }
    r.s0 = load_stat(a.stats + (size_t)row * a.S + min((int)threadIdx.x, a.S - 1));
}

// Resolve one row from its chunk summaries and candidates.  Runs in one workgroup of
// kThreads.  Returns false when the candidates cannot settle the row (the caller then
// runs dense_resolve).
// finish_list for lists of at most kThreads entries: the whole list sorted once (block
// rank sort), the top-p cut taken in it directly and the draw made over its kept
// prefix in vocab order; the same decisions as finish_list (the same fixed-point
// weights relative to the list's best score, the reference's exclusive rule within the
// crossing group of equal scores, the same rounding fallbacks), with fewer block phases.
// E[0..n) unsorted keys (n <= kThreads); W holds 2 * kThreads keys of scratch.
__device__ __forceinline__ bool finish_small(const Args &a, int row, int mode, const klsample_row_params &p,
                                             const unsigned long long *E, int n, bool topp, double zrow,
                                             bool complete, unsigned long long *W, Misc &ms) {
    const int V = a.V, N = a.N, tid = threadIdx.x;
    for (int i = tid; i < n; i += kThreads) W[i] = E[i];
    __syncthreads();
    if (n > 1) block_rank_sort(W, n, ms.part);
    __syncthreads();
    const float mref = desc_key_y(W[0]), ylo = desc_key_y(W[n - 1]);
    const unsigned long long zall = block_sumq(tid < n ? weight_fix(desc_key_y(W[tid]), mref) : 0ull, ms);
    TopPCut tc;
    bool cut_all = true;   // every entry kept
    if (topp) {
        const double target = (double)p.top_p * (zrow >= 0.0 ? zrow : (double)zall);
        if ((double)zall > target) {   // some entry's inclusive mass exceeds the target
            cut_in_sorted(W, n, 0ull, 0u, target, mref, tc, ms);
            cut_all = false;
        } else if (!complete) {
            return false;   // the kept mass reaches past the list
        }
    }
    const float cut = cut_all ? ylo : tc.cut;
    const int cut_idx = (cut_all || tc.cut_idx == 0x7fffffff) ? V : tc.cut_idx;
    const int kept_n = cut_all ? n : tc.kept;
    const unsigned long long zf = cut_all ? zall : tc.zf;
    // the kept prefix in vocab order, then the first entry whose inclusive mass exceeds
    // u * kept mass (the last one if rounding leaves it short)
    unsigned long long *X = W + kThreads;
    for (int i = tid; i < kept_n; i += kThreads)
        X[i] = ((unsigned long long)(uint32_t)desc_key_idx(W[i]) << 32) | __float_as_uint(desc_key_y(W[i]));
    __syncthreads();
    if (kept_n > 1) block_rank_sort(X, kept_n, ms.part);
    __syncthreads();
    const unsigned long long tgt = (unsigned long long)floor((double)p.uniform * (double)zf);
    if (wave_id() == 0) {
        const int l = lane_id();
        unsigned long long run = 0ull;
        int found = -1;
        for (int i0 = 0; i0 < kept_n && found < 0; i0 += 64) {
            const int i = i0 + l;
            const unsigned long long w = i < kept_n ? weight_fix(__uint_as_float((uint32_t)X[i]), mref) : 0ull;
            const unsigned long long incl = run + wave_incl_scan(w);
            const unsigned long long bal = __ballot(i < kept_n && incl > tgt);
            if (bal) found = i0 + __ffsll((long long)bal) - 1;
            run = readlane(incl, 63);
        }
        if (found < 0) found = max(kept_n - 1, 0);
        if (l == 0) ms.ia = found;
    }
    __syncthreads();
    const unsigned long long kt = X[ms.ia];
    RowOut r;
    r.token = (int)(kt >> 32);
    r.m = mref;
    r.cut = cut;
    r.cut_idx = cut_idx;
    r.kept = kept_n;
    r.log_norm = log((double)zf / kFixScale);
    r.logprob = (double)__uint_as_float((uint32_t)kt) - (double)mref - r.log_norm;
    r.path = 0;
    __syncthreads();
    emit_row(a, row, mode, r, W, min(N, kept_n), ms);   // the top-N: the sorted list's first entries
    return true;
}

template <typename TIn, int E>
__device__ __forceinline__ bool combine_row(const Args &a, int row, const klsample_row_params &p, int mode,
                                            const RowSpec &rs, unsigned char *raw, int *cnt, Misc &ms) {
    constexpr int C = kThreads * E;
    const int S = a.S, V = a.V, N = a.N;
    const int tid = threadIdx.x;
    const ChunkStat *st = a.stats + (size_t)row * S;
    const Cand *rc = a.cands + (size_t)row * S * a.cand_cap;

    // 1. The chunk summaries and the first candidate pairs of the first chunks (requested
    //    by the caller, request_row)
    int ppc, pshift, nspec;
    spec_layout(a, ppc, pshift, nspec);
    const uint4 *spec = rs.spec;
    const bool has = tid < S;
    const ChunkStat s0 = rs.s0;

    // 2. Row max, candidate bound, finite count, overflow (bit 0) and whether any chunk
    //    has candidates past the requested slots (bit 1); then sum-exp and argmax.
    float m = kNegInf, lo = kNegInf;
    int nfinite = 0, ovf = 0;
    if (has) {
        m = s0.m; lo = s0.y_thr; nfinite = s0.nfinite; ovf = s0.flags & kChunkOverflow;
        const int nc = min(s0.ncand, a.cand_cap);
        cnt[tid] = nc;
        if (tid >= nspec ? nc > 0 : nc > 2 * ppc) ovf |= 2;
    }
    for (int c = tid + kThreads; c < S; c += kThreads) {
        const ChunkStat s = st[c];
        m = fmaxf(m, s.m);
        lo = fmaxf(lo, s.y_thr);
        nfinite += s.nfinite;
        ovf |= s.flags & kChunkOverflow;
        const int nc = min(s.ncand, a.cand_cap);
        cnt[c] = nc;
        if (c >= nspec ? nc > 0 : nc > 2 * ppc) ovf |= 2;
    }
    ms.hist[tid] = 0u;   // kThreads == 256 bins, used by the selection below
    m = wave_reduce(m, OpMaxF(), kNegInf);
    lo = wave_reduce(lo, OpMaxF(), kNegInf);
    nfinite = wave_reduce(nfinite, OpSumI(), 0);
    ovf = wave_reduce(ovf, OpOrI(), 0);
    if (lane_id() == 0) {
        ms.rf[0][wave_id()] = m; ms.rf[1][wave_id()] = lo;
        ms.ri[0][wave_id()] = nfinite; ms.ri[1][wave_id()] = ovf;
    }
    if (tid == 0) { ms.ncand = 0; ms.ia = 0x7fffffff; ms.ib = 0; ms.ne = 0; ms.kmin = 0xffffffffu; ms.kmax = 0u; }
    __syncthreads();
    m = ms.rf[0][0]; lo = ms.rf[1][0]; nfinite = ms.ri[0][0]; ovf = ms.ri[1][0];
#pragma unroll
    for (int w = 1; w < kWaves; ++w) {
        m = fmaxf(m, ms.rf[0][w]); lo = fmaxf(lo, ms.rf[1][w]);
        nfinite += ms.ri[0][w]; ovf |= ms.ri[1][w];
    }
    if (ovf & 1) return false;   // a chunk's candidates overflowed (massive ties)
    const bool need_rest = (ovf & 2) != 0;
    int arg = 0x7fffffff;
    double Z = 0.0;
    if (mode != kTopK) {
        if (has) {
            if (mode == kGreedy && s0.m == m) arg = s0.arg;
            if (s0.m > kNegInf) Z += s0.z * (double)exp_fast(s0.m - m);
        }
        for (int c = tid + kThreads; c < S; c += kThreads) {
            const ChunkStat s = st[c];
            if (mode == kGreedy && s.m == m) arg = min(arg, s.arg);
            if (s.m > kNegInf) Z += s.z * (double)exp_fast(s.m - m);
        }
    }

    // A greedy row with no top-N list needs nothing but the summaries: argmax, and the
    // max and sum-exp of its logprob.
    if (mode == kGreedy && N == 0) {
        arg = wave_reduce(arg, OpMinI(), 0x7fffffff);
        Z = wave_reduce(Z, OpSumD(), 0.0);
        if (lane_id() == 0) {
            ms.red.d[wave_id()] = Z;
            atomicMin(&ms.ia, arg);
        }
        __syncthreads();
        Z = ms.red.d[0];
#pragma unroll
        for (int w = 1; w < kWaves; ++w) Z += ms.red.d[w];
        RowOut r;
        r.path = 0;
        r.m = m;
        r.cut = kNegInf;
        r.cut_idx = V;
        r.kept = nfinite;
        r.log_norm = log(Z);
        r.token = (ms.ia == 0x7fffffff) ? 0 : ms.ia;
        r.logprob = -r.log_norm;
        emit_row(a, row, mode, r, reinterpret_cast<unsigned long long *>(raw) + kSortCap, 0, ms);
        return true;
    }

    // 3. F = { candidates >= lo } into A; every element of the row scoring >= lo is in
    //    it.  Its key range is tracked for the selection.  Top-k rows keep their
    //    candidates' scores before the division by T (the order is the same): they are
    //    compared with xs, the smallest such score whose quotient reaches lo, and only
    //    the final top set is divided.
    unsigned long long *A = reinterpret_cast<unsigned long long *>(raw);
    unsigned long long *D = A + kSortCap;
    const float xs = (mode == kTopK) ? quotient_threshold(lo, p.temperature) : lo;
    uint32_t kmin = 0xffffffffu, kmax = 0u;
    {
        // the requested slots: accepted ones counted first, one LDS atomic per wave
        // reserves their places, then they are written
        uint32_t acc = 0u;
        // slot rounds whose first chunk is past the requested ones are skipped by the
        // whole wave
        const int wq0 = __builtin_amdgcn_readfirstlane(wave_id() * 64);
        int ncs[kSpecLoads];
#pragma unroll
        for (int i = 0; i < kSpecLoads; ++i)   // all counts read before any is used
            ncs[i] = cnt[min((tid + i * kThreads) >> pshift, kMaxChunksLds - 1)];
#pragma unroll
        for (int i = 0; i < kSpecLoads; ++i) {
            if (((wq0 + i * kThreads) >> pshift) >= nspec) break;
            const int q = tid + i * kThreads;
            const int nc = ((q >> pshift) < nspec) ? ncs[i] : 0, j = 2 * (q & (ppc - 1));
            if (j < nc && __uint_as_float(spec[i].x) >= xs) acc |= 1u << (2 * i);
            if (j + 1 < nc && __uint_as_float(spec[i].z) >= xs) acc |= 2u << (2 * i);
        }
        const int mine = __popc(acc);
        const int incl = wave_incl_scan(mine);
        int base = 0;
        if (lane_id() == 63 && incl > 0) base = atomicAdd(&ms.ncand, incl);
        base = readlane(base, 63) + incl - mine;
        // branch-free: every slot is stored, the rejected ones (and any past the list's
        // capacity) to the thread's sink; a taken branch per slot costs more
        unsigned long long *const sink = &ms.sink[tid];
        auto put = [&](bool ok, float y, int idx) {
            unsigned long long *dst = (ok && base < kSortCap) ? &A[base] : sink;
            *dst = desc_key(y, idx);
            base += ok ? 1 : 0;
            const uint32_t k = fkey(y);
            kmin = ok ? min(kmin, k) : kmin;
            kmax = ok ? max(kmax, k) : kmax;
        };
#pragma unroll
        for (int i = 0; i < kSpecLoads; ++i) {
            if (((wq0 + i * kThreads) >> pshift) >= nspec) break;
            put((acc >> (2 * i)) & 1u, __uint_as_float(spec[i].x), (int)spec[i].y);
            put((acc >> (2 * i + 1)) & 1u, __uint_as_float(spec[i].z), (int)spec[i].w);
        }
    }
    if (need_rest) {
        // the rest: chunks beyond the requested ones, and slots past the requested pairs.
        // Top-k rows: while more than 128 remain, eight slots per lane are requested at once
        // (clamped addresses), the accepted ones counted and their places reserved with one
        // LDS atomic per wave; the last ones (and every slot of other rows) are taken one
        // slot per lane at a time.
        const int l = lane_id();
        unsigned long long *const sink = &ms.sink[tid];
        auto visit = [&](auto width, const uint2 *pc, int j0, int nc) {
            constexpr int U = decltype(width)::value;
            uint2 e[U];
#pragma unroll
            for (int u = 0; u < U; ++u) e[u] = pc[min(j0 + u * 64 + l, nc - 1)];
            uint32_t acc = 0u;
#pragma unroll
            for (int u = 0; u < U; ++u)
                if (j0 + u * 64 + l < nc && __uint_as_float(e[u].x) >= xs) acc |= 1u << u;
            if (__ballot(acc != 0u) == 0ull) return;   // none accepted: nothing to store
            const int mine = __popc(acc);
            const int incl = wave_incl_scan(mine);
            int base = 0;
            if (l == 63) base = atomicAdd(&ms.ncand, incl);
            base = readlane(base, 63) + incl - mine;
#pragma unroll
            for (int u = 0; u < U; ++u) {   // branch-free, as for the requested slots
                const bool ok = (acc >> u) & 1u;
                const float y = __uint_as_float(e[u].x);
                *((ok && base < kSortCap) ? &A[base] : sink) = desc_key(y, (int)e[u].y);
                base += ok ? 1 : 0;
                const uint32_t k = fkey(y);
                kmin = ok ? min(kmin, k) : kmin;
                kmax = ok ? max(kmax, k) : kmax;
            }
        };
        for (int c = wave_id(); c < S; c += kWaves) {
            const int nc = cnt[c];
            const uint2 *pc = reinterpret_cast<const uint2 *>(rc + (size_t)c * a.cand_cap);
            int j0 = (c < nspec ? 2 * ppc : 0);
            if (mode == kTopK)
                for (; nc - j0 > 128; j0 += 512) visit(std::integral_constant<int, 8>{}, pc, j0, nc);
            for (int j = j0 + l; j < nc; j += 64) {   // the last 128 or fewer, one slot at a time
                const uint2 cd = pc[j];
                const float y = __uint_as_float(cd.x);
                if (y >= xs) {
                    const int pos = wave_append(&ms.ncand);
                    if (pos < kSortCap) A[pos] = desc_key(y, (int)cd.y);
                    const uint32_t k = fkey(y);
                    kmin = min(kmin, k);
                    kmax = max(kmax, k);
                }
            }
        }
    }
    // (the argmax serves greedy rows only, the sum-exp all but top-k rows)
    if (mode == kGreedy) arg = wave_reduce(arg, OpMinI(), 0x7fffffff);
    if (mode != kTopK) Z = wave_reduce(Z, OpSumD(), 0.0);
    kmin = wave_reduce(kmin, OpMinU(), 0xffffffffu);
    kmax = wave_reduce(kmax, OpMaxU(), 0u);
    if (lane_id() == 0) {
        ms.red.d[wave_id()] = Z;
        atomicMin(&ms.ia, arg);
        atomicMin(&ms.kmin, kmin);
        atomicMax(&ms.kmax, kmax);
    }
    __syncthreads();
    Z = ms.red.d[0];
#pragma unroll
    for (int w = 1; w < kWaves; ++w) Z += ms.red.d[w];
    arg = ms.ia;
    int nF = ms.ncand;
    float ylo = fkey_inv(ms.kmin), yhi = fkey_inv(ms.kmax);
    const bool narrowed = nF > kSortCap;   // the radix narrowing below leaves ms.hist used
    if (nF > kSortCap) {
        // Too many candidates for LDS: narrow them to the best R.  First a 256-bin
        // histogram over [ylo, yhi] (two passes over the candidate slots): the entries in
        // the bins at or above the R-th's, if they fit; else a radix select over the slots
        // (four passes) for the R-th and the entries scoring at least it.
        const int R = (mode == kTopK) ? p.top_k : (mode == kTopP ? kThreads : N);
        if (R < 1 || R > kSortCap) return false;
        const CandSource src{rc, cnt, S, a.cand_cap, xs};
        const float span = yhi - ylo, scale = 256.f / span;
        int t = -1;
        if (span > 0.f && scale <= __FLT_MAX__) {
            auto bin = [&](float y) { return min(255, (int)((y - ylo) * scale)); };
            ms.hist[tid] = 0u;   // kThreads == 256 bins
            __syncthreads();     // (every wave has read the candidate count)
            if (tid == 0) ms.ncand = 0;
            src.each([&](uint32_t, int, float y) { atomicAdd(&ms.hist[bin(y)], 1u); });
            __syncthreads();
            // the R-th from the top: every wave finds its bin from the same histogram
            const int l = lane_id();
            uint32_t c[4], sum = 0u;
#pragma unroll
            for (int j = 0; j < 4; ++j) { c[j] = ms.hist[255 - 4 * l - j]; sum += c[j]; }
            const uint32_t incl = wave_incl_scan(sum);
            const unsigned long long reach = __ballot(incl >= (uint32_t)R);
            const int fl = reach ? __ffsll((long long)reach) - 1 : 63;
            int b = 0;
            if (l == fl) {
                uint32_t acc = incl - sum;
                b = 252 - 4 * l;
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    if (acc + c[j] >= (uint32_t)R) { b = 255 - 4 * l - j; break; }
                    acc += c[j];
                }
            }
            b = __builtin_amdgcn_readlane(b, fl);
            src.each([&](uint32_t, int idx, float y) {
                if (bin(y) >= b) {
                    const int pos = wave_append(&ms.ncand);
                    if (pos < kSortCap) A[pos] = desc_key(y, idx);
                }
            });
            __syncthreads();
            t = ms.ncand;
        }
        if (t >= R && t <= kSortCap) {
            nF = t;
        } else {
            ylo = fkey_inv(select_kth(src, (uint32_t)R, ms));
            nF = gather_keys(src, ylo, A, kSortCap, ms);
            if (nF > kSortCap) return false;
        }
    }
    // D[0..n) := the best R of F (ties with the R-th included), sorted best first
    auto best = [&](int R) -> int {
        if (R < nF) return select_top(A, nF, R, ylo, yhi, D, kSortCap, ms);
        for (int i = tid; i < nF; i += kThreads) D[i] = A[i];
        __syncthreads();
        sort_top(D, nF, ms);
        return nF;
    };

    if (mode == kGreedy || mode == kFull) {
        const int want = min(N, nF);
        if (want > 0 && best(want) < 0) return false;
        RowOut r;
        r.path = 0;
        r.m = m;
        r.cut = kNegInf;
        r.cut_idx = V;
        r.kept = nfinite;
        r.log_norm = log(Z);
        if (mode == kGreedy) {
            r.token = (arg == 0x7fffffff) ? 0 : arg;
            r.logprob = -r.log_norm;
            emit_row(a, row, mode, r, D, want, ms);
            return true;
        }
        // full distribution: chunk-level inverse CDF, then an ordered rescan of the
        // chosen chunk (the top-N list moves out of the LDS the rescan reuses)
        for (int t = tid; t < want; t += kThreads) {
            ms.topn_idx[t] = desc_key_idx(D[t]);
            ms.topn_y[t] = desc_key_y(D[t]);
        }
        __syncthreads();
        const double target = (double)p.uniform * Z;
        int lastc;
        double before;
        int c = ordered_find(
            S, [&](int i) { const ChunkStat s = st[i]; return s.m > kNegInf ? s.z * exp((double)s.m - (double)m) : 0.0; },
            target, ms, lastc, before);
        if (c < 0) c = lastc >= 0 ? lastc : 0;
        const ChunkStat sc = st[c];
        const int c0 = c * C, cn = min(C, V - c0);
        const bool pen = has_penalty(a, p, row);
        uint32_t *ctab = reinterpret_cast<uint32_t *>(raw);
        __syncthreads();
        if (pen) build_counts<C>(ctab, a, row, c0, cn);
        const double scale = exp((double)sc.m - (double)m);
        const double rem = (target - before) / scale;
        int lastj;
        double bj;
        int j = ordered_find(
            cn, [&](int i) {
                const float y = element_final<TIn>(a, p, row, c0 + i, pen ? ctab : nullptr, c0, true);
                return (double)exp_fast(y - sc.m);
            },
            rem, ms, lastj, bj);
        if (j < 0) j = lastj >= 0 ? lastj : 0;
        r.token = c0 + j;
        const float yt = element_final<TIn>(a, p, row, r.token, pen ? ctab : nullptr, c0, true);
        r.logprob = (double)yt - (double)m - r.log_norm;
        __syncthreads();
        write_row(a, row, mode, r, want, ms);
        return true;
    }

    if (nF == 0) {
        // every score is -inf: nothing can be drawn
        RowOut r;
        r.path = 0; r.m = m; r.cut = kNegInf; r.cut_idx = V; r.kept = 0; r.log_norm = 0.0;
        r.token = 0; r.logprob = __builtin_nan("");
        write_row(a, row, mode, r, 0, ms);
        return true;
    }

    if (mode == kTopK) {
        // top-k: the kk best and every tie of the kk-th, then top-p on them.  The kk-th
        // largest score before division gives the kk-th quotient; the top set is every
        // candidate whose quotient reaches it (ties created by the division included),
        // divided and sorted in final space.
        const int kk = p.top_k;
        // the top set Es[0..lk) sorted in final space, with vocab-order ranks in ms.irank:
        // one wave applies top-p and finishes
        auto finish_top = [&](const unsigned long long *Es, int lk) {
            if (wave_id() == 0) {
                // the weights and one prefix scan serve the top-p cut and the kept sum
                const int l = lane_id();
                const float y0 = desc_key_y(Es[0]);
                const double mref = (double)y0;
                const double w = l < lk ? (double)__expf(desc_key_y(Es[l]) - y0) : 0.0;
                const double incl = wave_incl_scan(w);
                int L = lk;
                if (p.flags & KLSAMPLE_ROW_TOP_P) {
                    const double z = readlane(incl, lk - 1);
                    const unsigned long long cross = __ballot(l < lk && wave_shift_excl(incl) > (double)p.top_p * z);
                    if (cross) L = __ffsll((long long)cross) - 1;
                    if (L < 1) L = lk;
                }
                const double wz[2] = {w, readlane(incl, L - 1)};
                wave_finish(a, row, mode, p, Es, lk, L, mref, A, ms.irank, true, wz);
            }
        };
        int lk_pre = -1;   // the top set is D[0..lk_pre), sorted by score (set below)
        if (nF > kk && N <= 64) {
            // one histogram pass isolates the kk best; sorted, they give the kk-th
            // quotient, and the top set (every candidate whose quotient reaches it) is
            // gathered, divided and sorted; one wave applies top-p and finishes
            const int t = hist_gather(A, nF, kk, ylo, yhi, D, kSortCap, ms, narrowed);
            if (t >= kk && t <= 64) {
                // The gather holds the kk best and at most 64 entries in all: every wave
                // finds the kk-th best itself (the worst entry dropped t - kk times; no
                // barrier).  Every candidate scoring at least the smallest gathered score
                // is in the gather (its bin is at or above that one's), so when the kk-th
                // quotient's threshold xt is no lower than that score, the top set is the
                // gathered entries scoring >= xt.  -inf and signed zeros go the long way.
                const int l = lane_id();
                unsigned long long kl = l < t ? D[l] : 0ull;   // 0: never the worst
                unsigned long long kw = wave_reduce(kl, OpMaxQ(), 0ull);
                const float xmin = desc_key_y(kw);
                for (int r = kk; r < t; ++r) {
                    if (kl == kw) kl = 0ull;   // keys are distinct: drops one entry
                    kw = wave_reduce(kl, OpMaxQ(), 0ull);
                }
                const float xk = desc_key_y(kw);
                const float xt = (xk > kNegInf && xk != 0.f)
                                     ? quotient_threshold(__fdiv_rn(xk, p.temperature), p.temperature)
                                     : kNegInf;
                if (xk > kNegInf && xk != 0.f && xt >= xmin) {
                    const bool in = l < t && desc_key_y(D[l]) >= xt;
                    const unsigned long long bal = __ballot(in);
                    const int lk = __popcll(bal);
                    // final-space keys of the top set, into a copy (other waves may still
                    // be reading D)
                    const unsigned long long *Ef = D;
                    if (p.temperature != 1.f || lk < t) {
                        unsigned long long *Eq = D + 256;
                        if (wave_id() == 0 && in) {
                            const int pos = __builtin_amdgcn_mbcnt_hi((uint32_t)(bal >> 32),
                                                                      __builtin_amdgcn_mbcnt_lo((uint32_t)bal, 0u));
                            Eq[pos] = desc_key(__fdiv_rn(desc_key_y(D[l]), p.temperature), desc_key_idx(D[l]));
                        }
                        __syncthreads();
                        Ef = Eq;
                    }
                    const unsigned long long *Es = Ef;
                    if (lk > 1) {
                        unsigned long long *Eo = D + 128;
                        block_rank_sort_idx(Ef, lk, Eo, ms.part, ms.irank);
                        Es = Eo;
                    } else {
                        if (tid == 0) ms.irank[0] = 0u;
                        __syncthreads();
                    }
                    finish_top(Es, lk);
                    return true;
                }
            }
            if (t >= kk && t <= 256) {
                block_rank_sort(D, t, ms.part);
                const float xt = quotient_threshold(__fdiv_rn(desc_key_y(D[kk - 1]), p.temperature), p.temperature);
                const float xlast = desc_key_y(D[t - 1]);   // (read before D may be rewritten)
                unsigned long long *Et = D + 256;
                for (int i = tid; i < nF; i += kThreads) {
                    const unsigned long long k = A[i];
                    const float x = desc_key_y(k);
                    if (x >= xt) {
                        const int pos = wave_append(&ms.ne);
                        if (pos < 64) Et[pos] = desc_key(__fdiv_rn(x, p.temperature), desc_key_idx(k));
                    }
                }
                __syncthreads();
                const int lk = ms.ne;
                if (lk <= 64) {
                    // sorted (into D + 128) with every entry's vocab-order rank; one wave
                    // applies top-p and finishes
                    unsigned long long *Es = Et;
                    if (lk > 1) {
                        Es = D + 128;
                        block_rank_sort_idx(Et, lk, Es, ms.part, ms.irank);
                    } else if (tid == 0) {
                        ms.irank[0] = 0u;
                    }
                    if (lk <= 1) __syncthreads();
                    finish_top(Es, lk);
                    return true;
                }
                // more than 64 reach the k-th quotient: when every candidate reaching it
                // is in the sorted gather (its threshold is no lower than the gather's
                // smallest score), the top set is the gather's first lk entries
                if (xt >= xlast && lk <= t) lk_pre = lk;
            }
        }
        int lk = lk_pre;
        if (lk < 0) {
            float xt = kNegInf;
            if (nF > kk) {
                // the kk-th largest score by radix select: the top set is every candidate
                // whose quotient reaches its quotient
                const float xk = fkey_inv(select_kth(LdsSource{A, nF}, (uint32_t)kk, ms));
                xt = quotient_threshold(__fdiv_rn(xk, p.temperature), p.temperature);
            }
            lk = gather_ge(A, nF, xt, D, kSortCap, ms);
            if (lk > kSortCap) return false;
        }
        const bool topp = (p.flags & KLSAMPLE_ROW_TOP_P) != 0;
        const bool small = lk <= 64 && N <= 64;
        if (lk_pre < 0 || p.temperature != 1.f) {
            // divided into final space; sorted when the one-wave finish takes it (a
            // gather already sorted at T = 1 stays)
            for (int i = tid; i < lk; i += kThreads) {
                const unsigned long long k = D[i];
                D[i] = desc_key(__fdiv_rn(desc_key_y(k), p.temperature), desc_key_idx(k));
            }
            __syncthreads();
            if (small) sort_top(D, lk, ms);
        }
        if (!small) {
            if (lk <= kThreads) return finish_small(a, row, mode, p, D, lk, topp, -1.0, true, A, ms);
            return finish_list(a, row, mode, p, D, lk, topp, -1.0, true, A, ms);
        }
        const double mref = (double)desc_key_y(D[0]);
        if (wave_id() == 0) {
            int L = lk;
            if (topp) {
                const double w = lane_id() < lk ? (double)__expf(desc_key_y(D[lane_id()]) - (float)mref) : 0.0;
                const int cut = wave_topp(D, lk, mref, wave_reduce(w, OpSumD(), 0.0), p.top_p);
                if (cut > 0) L = cut;
            }
            wave_finish(a, row, mode, p, D, lk, L, mref, A);
        }
        return true;
    }

    // top-p alone: the best 48 or 64 (one wave), else every candidate (finish_list)
    const double mref = (double)m;
    if (nF > 64 && N <= 64) {
        // First the best 48 (and the ties of their bin): when that is at most 64 entries
        // they are sorted with their vocab-order ranks in one block pass and one wave
        // applies top-p and finishes (entries past the cut draw with weight 0), if the
        // kept set lies within them.  Otherwise the best 64 below.
        bool dirty = narrowed;
        if (nF > kTopPShort) {
            const int t = hist_gather(A, nF, kTopPShort, ylo, yhi, D, kSortCap, ms, dirty);
            dirty = true;
            if (t >= 2 && t <= 64) {
                unsigned long long *Eo = D + 128;
                block_rank_sort_idx(D, t, Eo, ms.part, ms.irank);
                if (wave_id() == 0) {
                    const int cut = wave_topp(Eo, t, mref, Z, p.top_p);
                    if (cut > 0) wave_finish(a, row, mode, p, Eo, t, cut, mref, A, ms.irank, true);
                    if (lane_id() == 0) ms.flag = cut;
                }
                __syncthreads();
                if (ms.flag > 0) return true;
            }
        }
        if (dirty) {
            __syncthreads();   // every wave has read the first gather's count
            if (threadIdx.x == 0) ms.ib = 0;   // hist_gather's counter
            __syncthreads();
        }
        const int t = hist_gather(A, nF, 64, ylo, yhi, D, kSortCap, ms, dirty);
        if (t >= 0 && t <= 256) {
            block_rank_sort(D, t, ms.part);
            if (wave_id() == 0) {
                const int cut = wave_topp(D, min(t, 64), mref, Z, p.top_p);
                if (lane_id() == 0) ms.flag = cut;
            }
            __syncthreads();
            const int cut = ms.flag;
            if (cut > 0) {
                block_index_rank(D, cut, ms.part, ms.irank);
                if (wave_id() == 0) wave_finish(a, row, mode, p, D, t, cut, mref, A, ms.irank);
                return true;
            }
        }
    }
    if (nF > 64 || N > 64) {
        // a kept set past the best 64 (or a long top-N list): from the unsorted candidates
        // (the kept set must lie within them unless they are the whole row)
        return finish_list(a, row, mode, p, A, nF, true, Z * kFixScale, !(lo > kNegInf), D, ms);
    }
    const int n = best(nF);
    if (n < 0) return false;
    if (wave_id() == 0) {
        const int cut = wave_topp(D, n, mref, Z, p.top_p);
        if (lane_id() == 0) ms.flag = cut;
    }
    __syncthreads();
    int L = ms.flag;
    if (L < 0) {
        if (lo > kNegInf) return false;   // the kept mass reaches past the candidates
        L = n;                            // the candidates are the whole row
    }
    if (wave_id() == 0) wave_finish(a, row, mode, p, D, n, L, mref, A);
    return true;
}

__device__ __forceinline__ void map_block(const Args &a, int w, int &row, int &chunk) {
    if (a.xcd_map) {
        // consecutive workgroup ids go to consecutive XCDs: keep a row's chunks on one
        // XCD so the row's history is fetched into one L2
        const int xcd = w & 7, slot = w >> 3;
        row = xcd + 8 * (slot / a.S);
        chunk = slot % a.S;
    } else {
        row = w / a.S;
        chunk = w % a.S;
    }
}

// LDS of the streaming pass.  Penalty phase: the chunk's history counts (16 bits, two
// per word), per thread a mask of its register slots holding a history element, and
// per wave a staging area where up to kStageLanes lanes at a time spill their
// registers to penalise them.  Later, the fallback bound's group keys.
constexpr int kStageLanes = 16;

template <int E>
struct ScanLds {
    static constexpr int C = kThreads * E;
    static constexpr int counts = C * 2;
    static constexpr int stride = E + 4;   // floats per staged lane (padded against bank conflicts)
    static constexpr int stage_off = counts;
    static constexpr int mask_off = stage_off + kWaves * kStageLanes * stride * 4;
    static constexpr int penalty = mask_off + kThreads * 4;
    static constexpr int keys = kThreads * (E < 16 ? E : 16) * 4;   // fallback bound (later)
    static constexpr int wide = kWideBins * 8 + 64;                  // top-p chunk histogram (last)
    static constexpr int value0 = penalty > keys ? penalty : keys;
    static constexpr int value = value0 > wide ? value0 : wide;
};

// A top-p chunk's histogram and final scores, into the workspace.  Bin j = G -
// floor(y * kWideCells) with G = floor(mc * kWideCells), capped at the last bin (see
// internal.h); each histogram word adds 1 at bit kWideCountShift and the entry's weight
// exp(y - G / kWideCells) in units of 2^-kWideMassBits below it (integer sums: exact
// and independent of their order).  The words are stored as an inclusive prefix over
// the bins (word j: bins 0..j; the packed count and mass add together, the chunk's
// totals staying below their fields' limits), so that the mass above any bin is one
// load.  The scores go to the row's score buffer in vocab order (16-byte stores).  x
// holds the chunk's final scores, -inf past its end.  `raw` holds kWideBins * 8 + 64
// bytes of free LDS.
template <typename TIn, int E>
__device__ __forceinline__ void wide_chunk(const Args &a, int row, int chunk, const float (&x)[E], float mc,
                                           unsigned char *raw) {
    constexpr int VW = Loader<TIn>::VW;
    constexpr int NV = E / VW;
    constexpr int C = kThreads * E;
    static_assert(C <= (1 << (64 - kWideCountShift - 1)), "bin counts must fit above kWideCountShift");
    static_assert(kWideCountShift >= kWideMassBits + 14, "bin masses must stay below kWideCountShift");
    const int tid = threadIdx.x;
    const int c0 = chunk * C, cn = min(C, a.V - c0);
    unsigned long long *hb = reinterpret_cast<unsigned long long *>(raw);
    uint4 *h4 = reinterpret_cast<uint4 *>(raw);
    for (int i = tid; i < kWideBins / 2; i += kThreads) h4[i] = make_uint4(0u, 0u, 0u, 0u);
    float *yb = a.ybuf + (size_t)row * a.ypitch + c0;
#pragma unroll
    for (int v = 0; v < NV; ++v) {
        const int li = (v * kThreads + tid) * VW;
        if (li + VW <= cn) {
#pragma unroll
            for (int q = 0; q < VW; q += 4)
                *reinterpret_cast<float4 *>(yb + li + q) =
                    make_float4(x[v * VW + q], x[v * VW + q + 1], x[v * VW + q + 2], x[v * VW + q + 3]);
        } else {
#pragma unroll
            for (int e = 0; e < VW; ++e)
                if (li + e < cn) yb[li + e] = x[v * VW + e];
        }
    }
    __syncthreads();   // bins cleared
    const float G = floorf(mc * kWideCells);
    const float anchor = G * (1.f / kWideCells);
#pragma unroll
    for (int e = 0; e < E; ++e) {
        const float y = x[e];
        if (y > kNegInf) {
            const float d = G - floorf(y * kWideCells);
            const int j = d < (float)(kWideBins - 1) ? (int)d : kWideBins - 1;
            atomicAdd(&hb[j], (1ull << kWideCountShift) + weight_fix<kWideMassBits>(y, anchor));
        }
    }
    __syncthreads();
    // inclusive prefix: four consecutive bins per thread, then across threads
    static_assert(kWideBins == 4 * kThreads, "four bins per thread");
    unsigned long long w4[4], run = 0ull;
#pragma unroll
    for (int k = 0; k < 4; ++k) { run += hb[4 * tid + k]; w4[k] = run; }
    const unsigned long long incl = wave_incl_scan(run);
    unsigned long long *wt = hb + kWideBins;   // the four waves' totals
    if (lane_id() == 63) wt[wave_id()] = incl;
    __syncthreads();
    unsigned long long off = incl - run;
    for (int w = 0; w < wave_id(); ++w) off += wt[w];
    uint4 *gh = reinterpret_cast<uint4 *>(a.hist + ((size_t)row * a.S + chunk) * kWideBins) + 2 * tid;
    const unsigned long long o0 = w4[0] + off, o1 = w4[1] + off, o2 = w4[2] + off, o3 = w4[3] + off;
    gh[0] = make_uint4((uint32_t)o0, (uint32_t)(o0 >> 32), (uint32_t)o1, (uint32_t)(o1 >> 32));
    gh[1] = make_uint4((uint32_t)o2, (uint32_t)(o2 >> 32), (uint32_t)o3, (uint32_t)(o3 >> 32));
}

// Streaming pass: one workgroup per (row, chunk).  The LDS footprint (~26 KB at 32
// elements per thread) lets six workgroups share a CU, and the register budget is
// capped to match (80 VGPRs: six waves per SIMD; seven or eight for smaller chunks),
// to hide HBM latency.
//
// Penalties: the row's history ids are counted into an LDS table and mark their
// element in its owner's slot mask (atomics whose results nobody waits for).  A lane
// owning marked elements spills its registers to its wave's LDS staging area,
// penalises the marked ones there (one per set mask bit) and reloads them, so the
// dense work that follows (bound, candidates, sums) sees final scores everywhere
// with no per-element branch.
// kInline: a launch whose row parameters (and maybe history offsets) are in the kernel
// arguments (small batches); a separate instantiation keeps the branch out of the
// streaming pass's register budget.  kLds: the chunk's logits come from LDS (`lsrc`,
// fp32, the chunk's C entries), where the LM-head kernel computed them.
template <typename TIn, int E, bool kVec, bool kInline, bool kLds = false>
__device__ __forceinline__ void scan_chunk(const Args &a, int row, int chunk, unsigned char *raw, ScanMisc &ms,
                                           bool wide_only, const float *lsrc = nullptr) {
    constexpr int VW = Loader<TIn>::VW;
    constexpr int NV = E / VW;
    constexpr int C = kThreads * E;
    const klsample_row_params p = kInline ? a.inl_params[row] : a.params[row];
    const int V = a.V;
    const int tid = threadIdx.x;
    const int mode = row_mode(p, V);
    // a second workgroup of a top-p chunk (small grids): only the histogram and scores
    if (wide_only && (mode != kTopP || a.S > kWideMaxChunks)) return;
    const bool divided = (mode == kTopP || mode == kFull);   // scores stream in final space
    const int c0 = chunk * C;
    const int cn = min(C, V - c0);
    const TIn *src = reinterpret_cast<const TIn *>(a.logits) + (int64_t)row * a.row_stride + c0;
    if (tid == 0) ms.ncand = 0;

    // History of a penalised row.  Its first ids are requested before the logits, so
    // the count table is built while the logits are in flight.  Counts are 16-bit
    // halves of LDS words (exact below 65536 ids); longer histories take the 32-bit
    // path below.
    // (the offsets are requested with the parameters, not after them: one memory round
    // trip before the loads start)
    int h0, h1;
    hist_range<kInline>(a, row, h0, h1);
    if (!(p.flags & (KLSAMPLE_ROW_REPETITION | KLSAMPLE_ROW_PRESENCE_FREQUENCY))) h1 = h0;
    const int H = h1 - h0;
    // 16-bit counts (two per word) cover the chunk when no count can reach 65536;
    // longer histories count in 32 bits over each half of the chunk in turn
    const bool packed = H < 65536;
    uint32_t *tab = reinterpret_cast<uint32_t *>(raw);
    uint32_t *hmask = reinterpret_cast<uint32_t *>(raw + ScanLds<E>::mask_off);
    auto clear = [&]() {
        uint4 *t4 = reinterpret_cast<uint4 *>(raw);
#pragma unroll
        for (int i = tid; i < C / 8; i += kThreads) t4[i] = make_uint4(0u, 0u, 0u, 0u);
        hmask[tid] = 0u;
    };
    int hid[8];
    if (H > 0) {
        // clamped addresses, unpredicated loads: all eight stay in flight together
#pragma unroll
        for (int j = 0; j < 8; ++j) hid[j] = a.hist_ids[min(h0 + tid + j * kThreads, h1 - 1)];
        clear();
    }

    // Rows that cannot take 16-byte loads (unaligned, or a last chunk shorter than one
    // vector) run the kVec = false instantiation.  Otherwise every chunk takes the same
    // vector loads (fp32: through a buffer resource over the chunk, 32-bit offsets,
    // vectors past its end reading 0; bf16: addresses clamped to the last whole vector of
    // a partial chunk, which keeps its registers within budget): one load path, so the
    // history count below waits for the ids only, with the logits still in flight.
    // Positions past cn are masked after the count; the vector straddling cn (if any) is
    // re-read element by element (every thread of a partial chunk reads it, its owner
    // keeps it).
    float x[E];
    float ptail[VW];
    if (kVec) {
        // the chunk as a buffer resource: 32-bit offsets (one per thread, the vector's
        // stride uniform), and vectors past the chunk's end read 0 instead of being
        // clamped (they are masked below)
        if constexpr (sizeof(TIn) == 4) {
            const __amdgpu_buffer_rsrc_t lg = __builtin_amdgcn_make_buffer_rsrc(
                const_cast<TIn *>(src), (short)0, cn * (int)sizeof(TIn), kBufferRsrcWord3);
            const uint32_t vo = (uint32_t)tid * (uint32_t)(VW * sizeof(TIn));
#pragma unroll
            for (int v = 0; v < NV; ++v)
                Loader<TIn>::vec_rsrc(lg, vo, (uint32_t)(v * kThreads * VW * sizeof(TIn)), &x[v * VW]);
        } else {
            const int lastfull = (cn / VW - 1) * VW;
#pragma unroll
            for (int v = 0; v < NV; ++v) Loader<TIn>::vec(src + min((v * kThreads + tid) * VW, lastfull), &x[v * VW]);
        }
        if (cn < C) {
            const int ls = (cn / VW) * VW;
#pragma unroll
            for (int e = 0; e < VW; ++e) ptail[e] = Loader<TIn>::one(src + min(ls + e, cn - 1));
        }
    } else {
#pragma unroll
        for (int v = 0; v < NV; ++v) {
#pragma unroll
            for (int e = 0; e < VW; ++e) {
                const int li = (v * kThreads + tid) * VW + e;
                if constexpr (kLds) x[v * VW + e] = (li < cn) ? lsrc[li] : kNegInf;
                else x[v * VW + e] = (li < cn) ? Loader<TIn>::one(src + li) : kNegInf;
            }
        }
    }

    auto mask_partial = [&]() {
        if (kVec && cn < C) {
            const int ls = (cn / VW) * VW;
#pragma unroll
            for (int v = 0; v < NV; ++v) {
                const int li = (v * kThreads + tid) * VW;
#pragma unroll
                for (int e = 0; e < VW; ++e)
                    x[v * VW + e] = (li + e < cn) ? (li >= ls ? ptail[e] : x[v * VW + e]) : kNegInf;
            }
        }
    };
    if (H == 0) mask_partial();

    if (H > 0) {
        // Counts the history ids falling in [lo, lo + span) of the chunk and marks their
        // owners' slots.  The ids were loaded from clamped positions: h >= h1 marks a
        // repeat, not an id.
        auto count_part = [&](auto wide, unsigned lo, unsigned span, bool preloaded) {
            auto count = [&](int id, int h) {
                const unsigned rel = (unsigned)id - (unsigned)c0;   // negative ids wrap past cn
                if (h < h1 && rel < (unsigned)cn && rel - lo < span) {
                    const unsigned owner = (rel / VW) % kThreads;
                    const unsigned slot = (rel / (VW * kThreads)) * VW + rel % VW;
                    if constexpr (decltype(wide)::value) atomicAdd(&tab[rel - lo], 1u);
                    else atomicAdd(&tab[rel >> 1], 1u << ((rel & 1u) * 16u));
                    atomicOr(&hmask[owner], 1u << slot);
                }
            };
            int hb = h0 + tid;
            if (preloaded) {
#pragma unroll
                for (int j = 0; j < 8; ++j) count(hid[j], hb + j * kThreads);
                hb += 8 * kThreads;
            }
            for (; hb < h1; hb += 8 * kThreads) {
#pragma unroll
                for (int j = 0; j < 8; ++j) hid[j] = a.hist_ids[min(hb + j * kThreads, h1 - 1)];
#pragma unroll
                for (int j = 0; j < 8; ++j) count(hid[j], hb + j * kThreads);
            }
        };
        // Penalises the marked elements: rounds of at most kStageLanes owner lanes per
        // wave spill their registers to the wave's own staging area (a wave's LDS
        // accesses complete in order), update the marked slots there and reload.
        auto apply = [&](bool wide, unsigned lo) {
            const uint32_t mk = hmask[tid];
            uint64_t pend = __ballot(mk != 0u);
            float *stage = reinterpret_cast<float *>(raw + ScanLds<E>::stage_off) +
                           wave_id() * (kStageLanes * ScanLds<E>::stride);
            const uint64_t below = (1ull << lane_id()) - 1ull;
            while (pend) {
                const int rank = __popcll(pend & below);
                const bool mine = ((pend >> lane_id()) & 1ull) && rank < kStageLanes;
                if (mine) {
                    float *sl = stage + rank * ScanLds<E>::stride;
#pragma unroll
                    for (int v = 0; v < E / 4; ++v)
                        *reinterpret_cast<float4 *>(sl + 4 * v) = make_float4(x[4 * v], x[4 * v + 1], x[4 * v + 2], x[4 * v + 3]);
                    uint32_t m = mk;
                    while (m) {
                        const int e = __builtin_ctz(m);
                        m &= m - 1u;
                        const unsigned rel = (unsigned)(((e / VW) * kThreads + tid) * VW + e % VW);
                        uint32_t c;
                        if (wide) c = tab[rel - lo];
                        else c = (tab[rel >> 1] >> ((rel & 1u) * 16u)) & 0xffffu;
                        sl[e] = penalize(sl[e], c, p);
                    }
#pragma unroll
                    for (int v = 0; v < E / 4; ++v) {
                        const float4 q = *reinterpret_cast<const float4 *>(sl + 4 * v);
                        x[4 * v] = q.x; x[4 * v + 1] = q.y; x[4 * v + 2] = q.z; x[4 * v + 3] = q.w;
                    }
                }
                pend &= ~__ballot(mine);
            }
        };
        // 32-bit counts of half a chunk fill the table: two parts.  The first count
        // stays outside the loop, so that it waits for the history ids only, not for
        // the logits loaded after them.
        constexpr unsigned kHalf = C / 2;
        const int parts = packed ? 1 : 2;
        __syncthreads();   // table cleared
        if (packed) count_part(std::false_type{}, 0u, (unsigned)C, true);
        else count_part(std::true_type{}, 0u, kHalf, true);
        mask_partial();
#pragma unroll 1
        for (int part = 0; part < parts; ++part) {
            if (part > 0) {
                __syncthreads();
                clear();
                __syncthreads();
                count_part(std::true_type{}, kHalf, kHalf, false);
            }
            __syncthreads();
            apply(!packed, part * kHalf);
        }
    }
    if (divided) {
#pragma unroll
        for (int e = 0; e < E; ++e) x[e] = __fdiv_rn(x[e], p.temperature);
    }
    if (wide_only) {
        // the chunk max as the first workgroup takes it (wave maxima, then the largest)
        float mt = kNegInf;
#pragma unroll
        for (int e = 0; e < E; ++e) mt = fmaxf(mt, x[e]);
        const float mw = wave_reduce(mt, OpMaxF(), kNegInf);
        if (lane_id() == 0) ms.wm[wave_id()] = mw;
        __syncthreads();
        float mc = ms.wm[0];
#pragma unroll
        for (int w = 1; w < kWaves; ++w) mc = fmaxf(mc, ms.wm[w]);
        if (mc > kNegInf && fabsf(mc) < kWideMaxScore) wide_chunk<TIn, E>(a, row, chunk, x, mc, raw);
        return;
    }

    ChunkStat st;
    st.m = kNegInf;
    st.arg = 0x7fffffff;
    st.y_thr = kNegInf;
    st.ncand = 0;
    st.z = 0.0;
    st.flags = 0;
    st.nfinite = 0;
    if (mode != kTopK) {
        // per wave (no barrier): max, lowest argmax, sum of exp relative to the wave's
        // max, finite count; thread 0 combines the waves after a later barrier
        float mt = kNegInf;
#pragma unroll
        for (int e = 0; e < E; ++e) mt = fmaxf(mt, x[e]);
        const float mw = wave_reduce(mt, OpMaxF(), kNegInf);
        int at = 0x7fffffff;
        if (mode == kGreedy) {
#pragma unroll
            for (int v = 0; v < NV; ++v) {
                const int li = (v * kThreads + tid) * VW;
#pragma unroll
                for (int e = 0; e < VW; ++e)
                    if (x[v * VW + e] == mw && li + e < cn && li + e < at) at = li + e;
            }
            at = wave_reduce(at, OpMinI(), 0x7fffffff);
        }
        double z = 0.0;
        int nfin = 0;
        if (mw > kNegInf) {
#pragma unroll
            for (int e = 0; e < E; ++e) {
                z += (double)exp_fast(x[e] - mw);
                nfin += (x[e] > kNegInf) ? 1 : 0;
            }
        }
        z = wave_reduce(z, OpSumD(), 0.0);
        nfin = wave_reduce(nfin, OpSumI(), 0);
        if (lane_id() == 0) {
            ms.wm[wave_id()] = mw;
            ms.wz[wave_id()] = z;
            ms.wn[wave_id()] = nfin;
            ms.wa[wave_id()] = at;
        }
    }

    const int K = (mode == kGreedy || mode == kFull) ? a.N
                  : (mode == kTopK ? p.top_k : max(kTopPCandidates, a.N));
    bool wide = false;      // a wide top-p chunk (decided below)
    float mc = kNegInf;     // ... and its max
    if (K > 0) {
        float bound = kNegInf;
        if (K < cn) bound = chunk_bound<E>(x, K, cn, tab, ms);
        else __syncthreads();
        // candidates: elements >= thr; a finite threshold also excludes -inf scores
        float thr = -__FLT_MAX__;
        auto set_bound = [&](float b) {
            thr = -__FLT_MAX__;
            if (b > kNegInf) {
                thr = b;
                if (mode == kTopK) {
                    // widen by 8 ulps so every element whose quotient by T rounds to at
                    // least b / T is kept
                    const float d = fmaxf(fabsf(b) * 9.5367431640625e-07f, p.temperature * 7.174648137343064e-43f);
                    thr = b - d;
                }
            }
            st.y_thr = (mode == kTopK) ? (b > kNegInf ? __fdiv_rn(b, p.temperature) : kNegInf) : b;
        };
        set_bound(bound);
        // each wave reserves its run of slots (one LDS atomic); the total is known after
        // the barrier, before any store, so no barrier waits for the stores
        int my, pos, total;
        auto reserve = [&]() {
            my = 0;
#pragma unroll
            for (int e = 0; e < E; ++e) my += (x[e] >= thr) ? 1 : 0;
            const int incl = wave_incl_scan(my);
            const int wtot = readlane(incl, 63);
            int wbase = 0;
            if (lane_id() == 0 && wtot > 0) wbase = atomicAdd(&ms.ncand, wtot);
            wbase = readlane(wbase, 0);
            pos = wbase + incl - my;
            __syncthreads();
            total = ms.ncand;
        };
        reserve();
        if (total > a.cand_cap && K < cn) {
            // Too many for the slots: a wave with few finite elements (the short last
            // chunk) drags the per-wave bound down.  Once more with the block-wide bound
            // over the chunk's finest groups.
            __syncthreads();   // every thread has read the count
            if (tid == 0) ms.ncand = 0;
            const float b2 = block_group_bound_dispatch<E>(x, E < 16 ? E : 16, K, tab, ms);
            if (b2 > bound) set_bound(b2);
            reserve();
        }
        // scores are written as streamed: top-k rows in the penalised space (the row
        // kernel divides by T), the others in final space
        // the chunk's slots as a buffer resource: stores past the capacity are dropped by
        // the hardware's range check (an overflowed chunk's slots are never read anyway)
        Cand *out = a.cands + ((size_t)row * a.S + chunk) * a.cand_cap;
        const __amdgpu_buffer_rsrc_t slots =
            __builtin_amdgcn_make_buffer_rsrc(out, (short)0, a.cand_cap * (int)sizeof(Cand), kBufferRsrcWord3);
#pragma unroll
        for (int v = 0; v < NV; ++v) {
            const int li = (v * kThreads + tid) * VW;
#pragma unroll
            for (int e = 0; e < VW; ++e) {
                const float xv = x[v * VW + e];
                if (xv >= thr) {
                    const u32x2 cd = {__float_as_uint(xv), (uint32_t)(c0 + li + e)};
                    __builtin_amdgcn_raw_buffer_store_b64(cd, slots, (uint32_t)pos * (uint32_t)sizeof(Cand), 0, 0);
                    ++pos;
                }
            }
        }
        st.ncand = min(total, a.cand_cap);
        st.flags = total > a.cand_cap ? kChunkOverflow : 0;
        // Every chunk of a top-p row also writes its histogram and final scores (at the
        // end, or in a second workgroup on small grids), so that a row whose kept set
        // reaches past the candidates can be resolved from them (wide_resolve).  Every
        // thread takes the same decision.
        if (mode == kTopP && a.S <= kWideMaxChunks) {
            mc = ms.wm[0];
#pragma unroll
            for (int w = 1; w < kWaves; ++w) mc = fmaxf(mc, ms.wm[w]);
            wide = mc > kNegInf && fabsf(mc) < kWideMaxScore;
            if (wide) st.flags |= kChunkWide;
        }
    } else {
        __syncthreads();
    }
    if (tid == 0) {
        if (mode != kTopK) {
            float m = ms.wm[0];
#pragma unroll
            for (int w = 1; w < kWaves; ++w) m = fmaxf(m, ms.wm[w]);
            double z = 0.0;
            int nfin = 0, at = 0x7fffffff;
#pragma unroll
            for (int w = 0; w < kWaves; ++w) {
                if (ms.wm[w] > kNegInf) z += ms.wz[w] * (double)exp_fast(ms.wm[w] - m);
                nfin += ms.wn[w];
                if (ms.wm[w] == m) at = min(at, ms.wa[w]);
            }
            st.m = m;
            st.z = z;
            st.nfinite = nfin;
            if (mode == kGreedy) st.arg = (at == 0x7fffffff) ? 0x7fffffff : c0 + at;
        }
        a.stats[(size_t)row * a.S + chunk] = st;
    }
    if (wide && !a.wide_split) wide_chunk<TIn, E>(a, row, chunk, x, mc, raw);
    if (a.hist_errors != nullptr && chunk == 0) {
        // (on request) the history ids outside [0, V) of a penalised row, which the
        // counting above skipped: counted once per row, by its first chunk
        int bad = 0;
        for (int h = h0 + tid; h < h1; h += kThreads) bad += ((unsigned)a.hist_ids[h] >= (unsigned)V) ? 1 : 0;
        bad = block_sum(bad, ms);
        if (tid == 0) a.hist_errors[row] = (uint32_t)bad;
    }
}

// (a launch with inline parameters has at most KLSAMPLE_HOST_PARAMS_MAX_BATCH rows, a few
// workgroups per CU at most: its register budget is not traded for occupancy)
template <typename TIn, int E, bool kVec, bool kInline>
__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(kInline ? 4 : E >= 32 ? 6 : E >= 16 ? 7 : 8))) void scan_kernel(Args a) {
    __shared__ __attribute__((aligned(16))) unsigned char raw[ScanLds<E>::value];
    __shared__ ScanMisc ms;
    // blocks past B * S are the second workgroups of top-p chunks (a.wide_split)
    const bool wide_only = blockIdx.x >= (unsigned)(a.B * a.S);
    int row, chunk;
    map_block(a, wide_only ? (int)blockIdx.x - a.B * a.S : (int)blockIdx.x, row, chunk);
    scan_chunk<TIn, E, kVec, kInline>(a, row, chunk, raw, ms, wide_only);
}

template <int C>
struct RowLds {
    static constexpr int a = C * 4;
    static constexpr int b = 2 * kSortCap * 8;
    static constexpr int w = (kWideCross + kWideList) * 8;   // wide_resolve
    static constexpr int ab = a > b ? a : b;
    static constexpr int value = ab > w ? ab : w;
};

// Whether every chunk of the row wrote its histogram (and none overflowed its candidate
// slots).
__device__ __forceinline__ bool all_chunks_wide(const Args &a, int row, Misc &ms) {
    int b = 0;
    for (int c = threadIdx.x; c < a.S; c += kThreads) {
        const int32_t f = a.stats[(size_t)row * a.S + c].flags;
        b |= ((f & kChunkWide) == 0 || (f & kChunkOverflow) != 0) ? 1 : 0;
    }
    return block_or(b, ms) == 0;
}

// A row of wide top-p chunks: its max from the chunk summaries, its top-N list from the
// candidates (every entry of the top N scores at least the largest chunk bound), then
// wide_resolve.  Returns false if the row is left to dense_resolve.
__device__ __forceinline__ bool wide_row(const Args &a, int row, const klsample_row_params &p, int mode, unsigned char *raw, int *cnt,
                         Misc &ms) {
    const int S = a.S, N = a.N, tid = threadIdx.x;
    const ChunkStat *st = a.stats + (size_t)row * S;
    float m = kNegInf, lo = kNegInf;
    for (int c = tid; c < S; c += kThreads) {
        const ChunkStat sc = st[c];
        m = fmaxf(m, sc.m);
        lo = fmaxf(lo, sc.y_thr);
        cnt[c] = min(sc.ncand, a.cand_cap);
    }
    m = block_max(m, ms);
    lo = block_max(lo, ms);
    if (!(m > kNegInf)) return false;
    int want = 0;
    if (N > 0) {
        unsigned long long *A = reinterpret_cast<unsigned long long *>(raw);
        unsigned long long *D = A + kSortCap;
        const CandSource src{a.cands + (size_t)row * S * a.cand_cap, cnt, S, a.cand_cap, lo};
        __syncthreads();   // (the counts in cnt)
        const int nF = gather_keys(src, lo, A, kSortCap, ms);
        if (nF < 1) return false;
        want = min(N, nF);
        int t;
        if (nF <= kSortCap) {
            const LdsSource ls{A, nF};
            const float tau = fkey_inv(select_kth(ls, (uint32_t)want, ms));
            t = gather_keys(ls, tau, D, kSortCap, ms);
        } else {
            // more candidates than the list holds: the radix select over their slots
            const float tau = fkey_inv(select_kth(src, (uint32_t)want, ms));
            t = gather_keys(src, tau, D, kSortCap, ms);
            if (t > kSortCap) return false;
        }
        sort_keys(D, t, ms.part);
        for (int i = tid; i < want; i += kThreads) {
            ms.topn_idx[i] = desc_key_idx(D[i]);
            ms.topn_y[i] = desc_key_y(D[i]);
        }
    }
    __syncthreads();   // (the candidate counts in cnt are no longer needed)
    return wide_resolve(a, row, p, mode, m, want, raw, reinterpret_cast<unsigned long long *>(cnt), ms);
}

// One row in one workgroup: combine the chunk candidates, or run the multi-pass path.
// `raw` holds RowLds<C>::value bytes, `cnt` kMaxChunksLds ints.
template <typename TIn, int E>
__device__ __forceinline__ void row_body(const Args &a, int row, unsigned char *raw, int *cnt, Misc &ms) {
    // the row's first loads go out before its parameters arrive (which are read through
    // the vector memory path, so that waiting for them waits for nothing else)
    RowSpec rs;
    request_row(a, row, rs);
    const klsample_row_params p =
        (a.inline_flags & kInlineParams) ? a.inl_params[row] : load_params_vmem(a.params, row);
    const int mode = row_mode(p, a.V);
    const bool force = (a.options & KLSAMPLE_OPT_FORCE_DENSE) != 0;
    bool done = false;
    if (!force && a.S <= kMaxChunksLds) done = combine_row<TIn, E>(a, row, p, mode, rs, raw, cnt, ms);
    if (!done && mode == kTopP && !force && a.S <= kWideMaxChunks) {
        // a top-p row whose kept set reaches past the candidates: resolved chunk by
        // chunk from the histograms and scores its chunks wrote
        __syncthreads();   // the combine's LDS is reused
        if (all_chunks_wide(a, row, ms)) done = wide_row(a, row, p, mode, raw, cnt, ms);
    }
    if (!done) {
        __syncthreads();   // the combine's LDS (cnt included) is reused
        dense_resolve<TIn, E>(a, row, p, mode, raw, cnt, ms);
    }
}

template <typename TIn, int E>
__global__ __launch_bounds__(kThreads) void row_kernel(Args a) {
    constexpr int C = kThreads * E;
    __shared__ __attribute__((aligned(16))) unsigned char raw[RowLds<C>::value];
    __shared__ int cnt[kMaxChunksLds];
    __shared__ Misc ms;
    row_body<TIn, E>(a, blockIdx.x, raw, cnt, ms);
}

// ---------------------------------------------------------------------------------
// LM head fused with the streaming pass (serving/qwen_executor.py:238 computes
// lm_head(hidden) in bf16, then the sampler reads the logits back).  Workgroup
// (chunk, row block) multiplies its kThreads * kHeadElems vocabulary rows of the weight
// with kHeadRows hidden rows: each wave owns 256 vocabulary rows as sixteen 16x16 tiles
// of v_mfma_f32_16x16x32_bf16 (vocabulary along M, batch along N, 32 of the hidden
// dimension per step, the next step's operands loaded before this step's products).
// The fp32 sums are rounded to bf16 as the reference's bf16 output is, written to LDS
// and to the materialised logits, and each row of the block is then scanned from LDS by
// the streaming pass's own code.  The row kernel follows as for any call.
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));

__device__ __forceinline__ float round_bf16(float x) {
    uint32_t u = __float_as_uint(x);
    if ((u & 0x7fffffffu) > 0x7f800000u) return __uint_as_float(u | 0x00400000u);   // NaN stays NaN
    u += 0x7fffu + ((u >> 16) & 1u);                                                 // nearest, ties to even
    return __uint_as_float(u & 0xffff0000u);
}

template <bool kInline>
__global__ __launch_bounds__(kThreads) void lmhead_kernel(Args a, HeadArgs h) {
    constexpr int C = kThreads * kHeadElems;
    constexpr int kTiles = C / kWaves / 16;   // 16-row vocabulary tiles per wave
    __shared__ __attribute__((aligned(16))) float lg[kHeadRows * C];
    __shared__ __attribute__((aligned(16))) unsigned char raw[ScanLds<kHeadElems>::value];
    __shared__ ScanMisc ms;
    const int chunk = (int)blockIdx.x % a.S;
    const int r0 = ((int)blockIdx.x / a.S) * kHeadRows;
    const int w = wave_id(), l = lane_id();
    const int g = l >> 4, n = l & 15;          // lane group (8 of the 32 hidden entries a step), tile row / column
    const int vwave = chunk * C + w * (C / kWaves);
    // operand rows: vocabulary rows past V and batch rows past B read row 0 / a zero operand
    const uint16_t *wrow[kTiles];
#pragma unroll
    for (int t = 0; t < kTiles; ++t) {
        const int v = vwave + t * 16 + n;
        wrow[t] = h.weight + (size_t)(v < a.V ? v : 0) * h.dim + 8 * g;
    }
    // (rows past B repeat the block's last row: their products are neither scanned nor
    // written, and the loads stay unconditional)
    const uint16_t *hrow = h.hidden + (size_t)min(r0 + n, a.B - 1) * h.dim + 8 * g;
    f32x4 acc[kTiles];
#pragma unroll
    for (int t = 0; t < kTiles; ++t) acc[t] = f32x4{0.f, 0.f, 0.f, 0.f};
    // Two operand sets take turns, each reloaded two steps ahead right after its products
    // are issued: two steps of loads stay in flight.  Every load is unconditional (the
    // offsets clamp to the last step, dim being a multiple of 64), so that the waits
    // before the products count only the loads they need.
    bf16x8 ax[kTiles], ay[kTiles], bx, by;
    auto load = [&](bf16x8 (&av)[kTiles], bf16x8 &bv, int k) {
        k = min(k, h.dim - 32);
#pragma unroll
        for (int t = 0; t < kTiles; ++t) av[t] = *reinterpret_cast<const bf16x8 *>(wrow[t] + k);
        bv = *reinterpret_cast<const bf16x8 *>(hrow + k);
        __builtin_amdgcn_sched_barrier(0);   // the loads stay here, ahead of the products that need them
    };
    load(ax, bx, 0);
    load(ay, by, 32);
    for (int k0 = 0; k0 < h.dim; k0 += 64) {
#pragma unroll
        for (int t = 0; t < kTiles; ++t) acc[t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ax[t], bx, acc[t], 0, 0, 0);
        load(ax, bx, k0 + 64);
#pragma unroll
        for (int t = 0; t < kTiles; ++t) acc[t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ay[t], by, acc[t], 0, 0, 0);
        load(ay, by, k0 + 96);
    }
    // tile t, lane l, entry j: vocabulary row vwave + 16t + 4g + j, batch row r0 + n
    const int rowg = r0 + n;
#pragma unroll
    for (int t = 0; t < kTiles; ++t) {
        const int vl = w * (C / kWaves) + t * 16 + 4 * g;   // within the chunk
        const f32x4 q = {round_bf16(acc[t][0]), round_bf16(acc[t][1]), round_bf16(acc[t][2]), round_bf16(acc[t][3])};
        *reinterpret_cast<f32x4 *>(&lg[n * C + vl]) = q;
        const int v = chunk * C + vl;
        if (rowg < a.B) {
            float *o = h.logits_out + (size_t)rowg * a.V + v;
#pragma unroll
            for (int j = 0; j < 4; ++j)
                if (v + j < a.V) o[j] = q[j];
        }
    }
    __syncthreads();
    const int rows = min(kHeadRows, a.B - r0);
    for (int i = 0; i < rows; ++i) {
        scan_chunk<float, kHeadElems, false, kInline, true>(a, r0 + i, chunk, raw, ms, false, lg + i * C);
        __syncthreads();
    }
}

// Final probabilities: exp(s - max - log_norm) on the kept set, 0 elsewhere.
template <typename TIn, int E>
__global__ __launch_bounds__(kThreads) void probs_kernel(Args a) {
    constexpr int C = kThreads * E;
    __shared__ __attribute__((aligned(16))) uint32_t cnt[C];
    int row, chunk;
    map_block(a, blockIdx.x, row, chunk);
    const klsample_row_params p = row_params(a, row);
    const int mode = row_mode(p, a.V);
    const klsample_row_info ri = a.rows[row];
    const int c0 = chunk * C, cn = min(C, a.V - c0);
    const bool pen = has_penalty(a, p, row);
    if (pen) build_counts<C>(cnt, a, row, c0, cn);
    for (int i = threadIdx.x; i < cn; i += kThreads) {
        const int gi = c0 + i;
        const float y = element_final<TIn>(a, p, row, gi, pen ? cnt : nullptr, c0, mode != kGreedy);
        const bool kept = (mode == kGreedy || mode == kFull) ||
                          y > ri.cut_score || (y == ri.cut_score && gi <= ri.cut_index);
        const float pr = kept ? (float)exp((double)y - (double)ri.max_score - ri.log_norm) : 0.f;
        a.probs[(size_t)row * a.V + gi] = pr;
    }
}

__global__ void zero_fill_kernel(uint4 *p, size_t n16, unsigned char *tail, size_t ntail) {
    const size_t stride = (size_t)gridDim.x * blockDim.x;
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n16; i += stride)
        p[i] = make_uint4(0u, 0u, 0u, 0u);
    if (blockIdx.x == 0)
        for (size_t i = threadIdx.x; i < ntail; i += blockDim.x) tail[i] = 0;
}

hipError_t mark(const PhaseEvents *ph, int i, hipStream_t s) {
    if (ph == nullptr || ph->ev[i] == nullptr) return hipSuccess;
    return hipEventRecord(ph->ev[i], s);
}

template <typename TIn, int E>
hipError_t launch_typed(const Args &a, hipStream_t s, const PhaseEvents *ph) {
    const dim3 grid((unsigned)((int64_t)a.B * a.S));
    const dim3 scan_grid((unsigned)((int64_t)a.B * a.S * (a.wide_split ? 2 : 1)));
    hipError_t e = mark(ph, 0, s);
    if (e != hipSuccess) return e;
    // 16-byte loads need aligned rows and a last chunk of at least one vector
    const int tail = a.V - (a.S - 1) * a.C;
    const bool vec = a.vec_ok && tail * (int)sizeof(TIn) >= 16;
    if (a.inline_flags & kInlineParams) {
        if (vec) scan_kernel<TIn, E, true, true><<<scan_grid, kThreads, 0, s>>>(a);
        else scan_kernel<TIn, E, false, true><<<scan_grid, kThreads, 0, s>>>(a);
    } else {
        if (vec) scan_kernel<TIn, E, true, false><<<scan_grid, kThreads, 0, s>>>(a);
        else scan_kernel<TIn, E, false, false><<<scan_grid, kThreads, 0, s>>>(a);
    }
    if ((e = mark(ph, 1, s)) != hipSuccess) return e;
    row_kernel<TIn, E><<<dim3((unsigned)a.B), kThreads, 0, s>>>(a);
    if ((e = mark(ph, 2, s)) != hipSuccess) return e;
    if (a.probs) probs_kernel<TIn, E><<<grid, kThreads, 0, s>>>(a);
    if ((e = mark(ph, 3, s)) != hipSuccess) return e;
    return hipGetLastError();
}

}  // namespace

hipError_t launch_lmhead(const Args &a, const HeadArgs &h, hipStream_t s) {
    if (a.E != kHeadElems || a.wide_split) return hipErrorInvalidValue;
    const dim3 grid((unsigned)((int64_t)a.S * ((a.B + kHeadRows - 1) / kHeadRows)));
    if (a.inline_flags & kInlineParams) lmhead_kernel<true><<<grid, kThreads, 0, s>>>(a, h);
    else lmhead_kernel<false><<<grid, kThreads, 0, s>>>(a, h);
    row_kernel<float, kHeadElems><<<dim3((unsigned)a.B), kThreads, 0, s>>>(a);
    if (a.probs) probs_kernel<float, kHeadElems><<<dim3((unsigned)((int64_t)a.B * a.S)), kThreads, 0, s>>>(a);
    return hipGetLastError();
}

hipError_t launch_sample(const Args &a, int32_t dtype, hipStream_t s, const PhaseEvents *ph) {
    if (dtype == KLSAMPLE_FLOAT32) {
        switch (a.E) {
            case 4: return launch_typed<float, 4>(a, s, ph);
            case 8: return launch_typed<float, 8>(a, s, ph);
            case 16: return launch_typed<float, 16>(a, s, ph);
            case 32: return launch_typed<float, 32>(a, s, ph);
        }
    } else {
        switch (a.E) {
            case 8: return launch_typed<uint16_t, 8>(a, s, ph);
            case 16: return launch_typed<uint16_t, 16>(a, s, ph);
            case 32: return launch_typed<uint16_t, 32>(a, s, ph);
        }
    }
    return hipErrorInvalidValue;
}

// ---------------------------------------------------------------------------------
// The workspace of klsample_run_noalloc: one array per GPU, held until the process
// ends.  In host code `scratch` names a host-side stand-in, not device memory: its
// device address comes from hipGetSymbolAddress, taken once per device (with that
// device current) and kept, and only that address is handed to kernels.  No call
// needs the array cleared: every workspace byte a call reads was written earlier in
// the same call.  Calls that overlap on one GPU share it and race.
static __device__ __align__(256) unsigned char scratch[kScratchBytes];

constexpr int kScratchDevices = 64;

hipError_t scratch_workspace(hipStream_t s, void **ptr) {
    static std::mutex mu;
    static void *addr[kScratchDevices] = {};
    int dev = -1;
    hipError_t e = (s != nullptr) ? hipStreamGetDevice(s, &dev) : hipGetDevice(&dev);
    if (e != hipSuccess) return e;
    if (dev < 0 || dev >= kScratchDevices) return hipErrorInvalidDevice;
    std::lock_guard<std::mutex> lock(mu);
    if (addr[dev] == nullptr) {
        int cur = -1;
        if ((e = hipGetDevice(&cur)) != hipSuccess) return e;
        if (cur != dev && (e = hipSetDevice(dev)) != hipSuccess) return e;
        void *p = nullptr;
        e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (cur != dev) {
            const hipError_t back = hipSetDevice(cur);
            if (e == hipSuccess) e = back;
        }
        if (e != hipSuccess) return e;
        if (p == nullptr) return hipErrorInvalidSymbol;
        addr[dev] = p;
    }
    *ptr = addr[dev];
    return hipSuccess;
}

hipError_t launch_zero_fill(void *ptr, size_t bytes, hipStream_t s) {
    unsigned char *base = static_cast<unsigned char *>(ptr);
    const size_t head = (16 - ((uintptr_t)base & 15)) & 15;
    if (head) {
        zero_fill_kernel<<<1, 64, 0, s>>>(nullptr, 0, base, head < bytes ? head : bytes);
        if (head >= bytes) return hipGetLastError();
    }
    const size_t rest = bytes - head;
    const size_t n16 = rest / 16;
    const unsigned blocks = (unsigned)(n16 / 256 + 1 < 1024 ? n16 / 256 + 1 : 1024);
    zero_fill_kernel<<<blocks, 256, 0, s>>>(reinterpret_cast<uint4 *>(base + head), n16,
                                            base + head + n16 * 16, rest - n16 * 16);
    return hipGetLastError();
}

}  // namespace kls
