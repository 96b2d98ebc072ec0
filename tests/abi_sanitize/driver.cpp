// Drives every entry point of the C ABI (include/klsample.h) through its argument checks
// and its launch planning, with the launches replaced by stubs.cpp.  Built with
// -fsanitize=address,undefined by tests/test_abi_sanitize.py; prints "ok" and returns 0
// when every check holds.
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include <string>
#include <thread>
#include <vector>

#include "klsample.h"
#include "stubs.h"

static int failures = 0;
#define CHECK(cond)                                                           \
    do {                                                                      \
        if (!(cond)) {                                                        \
            fprintf(stderr, "check failed at line %d: %s\n", __LINE__, #cond); \
            ++failures;                                                       \
        }                                                                     \
    } while (0)

// host buffers standing in for device memory (the stubs never dereference them)
struct Bufs {
    std::vector<float> logits;
    std::vector<klsample_row_params> params;
    std::vector<int32_t> ids, off;
    std::vector<int64_t> tok;
    std::vector<float> lp, top_lp;
    std::vector<int32_t> top_ids;
    std::vector<unsigned char> ws;
    void *ws_aligned = nullptr;
    size_t ws_bytes = 0;
};

static klsample_batch make_batch(Bufs &b, int B, int V, int N, int32_t max_top_k) {
    b.logits.assign((size_t)B * V + 8, 0.f);
    b.params.assign(B, klsample_row_params{});
    b.ids.assign(16, 1);
    b.off.assign(B + 1, 0);
    b.off[B] = 16;
    b.tok.assign(B, 0);
    b.lp.assign(B, 0.f);
    b.top_ids.assign((size_t)B * (N > 0 ? N : 1), 0);
    b.top_lp.assign((size_t)B * (N > 0 ? N : 1), 0.f);
    size_t bytes = 0;
    CHECK(klsample_workspace_size(B, V, KLSAMPLE_FLOAT32, max_top_k, N, &bytes) == KLSAMPLE_OK);
    b.ws.assign(bytes + 256, 0);
    uintptr_t p = (uintptr_t)b.ws.data();
    b.ws_aligned = (void *)((p + 255) & ~(uintptr_t)255);
    b.ws_bytes = bytes;
    klsample_batch k;
    memset(&k, 0, sizeof k);
    k.logits = b.logits.data();
    k.row_stride = V;
    k.dtype = KLSAMPLE_FLOAT32;
    k.batch = B;
    k.vocab = V;
    k.num_logprobs = N;
    k.max_top_k = max_top_k;
    k.params = b.params.data();
    k.history_ids = b.ids.data();
    k.history_offsets = b.off.data();
    k.token_ids = b.tok.data();
    k.logprobs = b.lp.data();
    k.top_ids = N > 0 ? b.top_ids.data() : nullptr;
    k.top_logprobs = N > 0 ? b.top_lp.data() : nullptr;
    k.workspace = b.ws_aligned;
    k.workspace_bytes = b.ws_bytes;
    return k;
}

// every workspace region the launch received lies inside the workspace, 256-aligned
static void check_plan(const Bufs &b, const klsample_batch &k, bool head = false) {
    const kls::Args &a = stub::last_args;
    const uintptr_t lo = (uintptr_t)k.workspace, hi = lo + k.workspace_bytes;
    auto inside = [&](const void *p, size_t n) {
        const uintptr_t q = (uintptr_t)p;
        return q >= lo && q + n <= hi && (q & 255u) == 0;
    };
    const size_t BS = (size_t)a.B * a.S;
    CHECK(a.B == k.batch && a.V == k.vocab && a.N == k.num_logprobs);
    CHECK(a.C == 256 * a.E && (int64_t)a.S * a.C >= a.V && (int64_t)(a.S - 1) * a.C < a.V);
    CHECK(inside(a.stats, BS * sizeof(kls::ChunkStat)));
    CHECK(inside(a.cands, BS * (size_t)a.cand_cap * sizeof(kls::Cand)));
    CHECK(inside(a.rows, (size_t)a.B * sizeof(klsample_row_info)));
    CHECK(inside(a.ybuf, (size_t)a.B * a.ypitch * sizeof(float)));
    CHECK(inside(a.hist, BS * (size_t)kls::kWideBins * 8));
    CHECK(a.ypitch >= a.V + 1 && a.ypitch % 4 == 0);
    const int kk = k.max_top_k < a.V ? k.max_top_k : a.V;
    const int want = 2 * (kk > 64 ? kk : 64) + 128;   // slots for the chunk's K best, capped at the chunk
    CHECK(a.cand_cap >= (want < a.C ? want : a.C) && a.cand_cap <= a.C && a.cand_cap % 64 == 0);
    CHECK(a.wide_split == (!head && BS <= (size_t)kls::kWideSplitGroups ? 1 : 0));
    (void)b;
}

static void expect_error(const klsample_batch *k, int status) {
    const int st = klsample_run(k, nullptr);
    CHECK(st == status);
    CHECK(strlen(klsample_last_error()) > 0);
}

int main() {
    CHECK(klsample_abi_version() == KLSAMPLE_ABI_VERSION);

    // workspace sizes
    size_t bytes = 0;
    CHECK(klsample_workspace_size(0, 10, KLSAMPLE_FLOAT32, 0, 0, &bytes) == KLSAMPLE_ERR_INVALID_ARGUMENT);
    CHECK(klsample_workspace_size(1, 0, KLSAMPLE_FLOAT32, 0, 0, &bytes) == KLSAMPLE_ERR_INVALID_ARGUMENT);
    CHECK(klsample_workspace_size(1, 10, 7, 0, 0, &bytes) == KLSAMPLE_ERR_UNSUPPORTED_DTYPE);
    CHECK(klsample_workspace_size(1, 10, KLSAMPLE_FLOAT32, -1, 0, &bytes) == KLSAMPLE_ERR_INVALID_ARGUMENT);
    CHECK(klsample_workspace_size(1, 10, KLSAMPLE_FLOAT32, 0, 257, &bytes) == KLSAMPLE_ERR_INVALID_ARGUMENT);
    CHECK(klsample_workspace_size(1, 10, KLSAMPLE_FLOAT32, 0, 0, nullptr) == KLSAMPLE_ERR_INVALID_ARGUMENT);
    CHECK(klsample_workspace_size(1, 1 << 24, KLSAMPLE_BFLOAT16, 1 << 30, 256, &bytes) == KLSAMPLE_OK);
    CHECK(strlen(klsample_last_error()) == 0);

    // valid calls of several shapes: the plan handed to the launch stays in the workspace
    const int shapes[][4] = {{1, 151936, 0, 0}, {8, 151936, 5, 50}, {64, 151936, 20, 1000},
                             {3, 1, 0, 0}, {5, 70001, 256, 5000}, {256, 128256, 0, 40}};
    for (const auto &sh : shapes) {
        Bufs b;
        klsample_batch k = make_batch(b, sh[0], sh[1], sh[2], sh[3]);
        const int before = stub::launches;
        CHECK(klsample_run(&k, nullptr) == KLSAMPLE_OK);
        CHECK(stub::launches == before + 1);
        check_plan(b, k);
    }

    // argument errors, each reported before any launch
    {
        Bufs b;
        klsample_batch k = make_batch(b, 4, 1000, 3, 10);
        const int before = stub::launches;
        expect_error(nullptr, KLSAMPLE_ERR_INVALID_ARGUMENT);
        klsample_batch e = k; e.logits = nullptr; expect_error(&e, KLSAMPLE_ERR_INVALID_ARGUMENT);
        e = k; e.row_stride = 999; expect_error(&e, KLSAMPLE_ERR_INVALID_ARGUMENT);
        e = k; e.params = nullptr; expect_error(&e, KLSAMPLE_ERR_INVALID_ARGUMENT);
        e = k; e.token_ids = nullptr; expect_error(&e, KLSAMPLE_ERR_INVALID_ARGUMENT);
        e = k; e.top_ids = nullptr; expect_error(&e, KLSAMPLE_ERR_INVALID_ARGUMENT);
        e = k; e.history_ids = nullptr; expect_error(&e, KLSAMPLE_ERR_INVALID_ARGUMENT);
        e = k; e.options = 0x80u; expect_error(&e, KLSAMPLE_ERR_INVALID_ARGUMENT);
        e = k; e.dtype = 3; expect_error(&e, KLSAMPLE_ERR_UNSUPPORTED_DTYPE);
        e = k; e.batch = 0; expect_error(&e, KLSAMPLE_ERR_INVALID_ARGUMENT);
        e = k; e.workspace = nullptr; expect_error(&e, KLSAMPLE_ERR_WORKSPACE);
        e = k; e.workspace = (unsigned char *)k.workspace + 16; expect_error(&e, KLSAMPLE_ERR_WORKSPACE);
        e = k; e.workspace_bytes = k.workspace_bytes - 1; expect_error(&e, KLSAMPLE_ERR_WORKSPACE);
        CHECK(stub::launches == before);
        // the allocation-free entry point: no workspace accepted, size limit enforced
        CHECK(klsample_run_noalloc(&k, nullptr) == KLSAMPLE_ERR_WORKSPACE);
        e = k; e.workspace = nullptr; e.workspace_bytes = 0;
        CHECK(klsample_run_noalloc(&e, nullptr) == KLSAMPLE_OK);
        CHECK(stub::last_args.stats == (void *)stub::scratch);
        Bufs big;
        klsample_batch kb = make_batch(big, 4096, 151936, 0, 0);
        kb.workspace = nullptr; kb.workspace_bytes = 0;
        CHECK(klsample_run_noalloc(&kb, nullptr) == KLSAMPLE_ERR_WORKSPACE);
    }

    // host parameters: copied into the launch arguments (exact sizes, so that an overread
    // is caught), history offsets too; more than the inline rows is an argument error
    for (int B = 1; B <= KLSAMPLE_HOST_PARAMS_MAX_BATCH; B += 7) {
        for (int pairs = 0; pairs < 2; ++pairs) {
            Bufs b;
            klsample_batch k = make_batch(b, B, 5000, 2, 40);
            std::vector<klsample_row_params> hp(B);
            for (int i = 0; i < B; ++i) hp[i].top_k = 7 + i;
            std::vector<int32_t> ho(pairs ? 2 * B : B + 1);
            for (size_t i = 0; i < ho.size(); ++i) ho[i] = (int32_t)(3 * i);
            k.params = hp.data();
            k.history_offsets = ho.data();
            k.options = KLSAMPLE_OPT_HOST_PARAMS | (pairs ? KLSAMPLE_OPT_HISTORY_PAIRS : 0u);
            if (pairs) k.history_append = b.ids.data();
            CHECK(klsample_run(&k, nullptr) == KLSAMPLE_OK);
            const kls::Args &a = stub::last_args;
            CHECK(a.params == nullptr && a.hist_off == nullptr);
            CHECK(a.inline_flags == (kls::kInlineParams | kls::kInlineOffsets));
            CHECK(a.inl_params[B - 1].top_k == 7 + B - 1 && a.inl_off[ho.size() - 1] == ho.back());
            CHECK(a.hist_append == (pairs ? b.ids.data() : nullptr));
            k.history_offsets = nullptr;
            k.history_append = nullptr;
            CHECK(klsample_run(&k, nullptr) == KLSAMPLE_OK);
            CHECK(stub::last_args.inline_flags == kls::kInlineParams);
        }
    }
    {
        Bufs b;
        klsample_batch k = make_batch(b, KLSAMPLE_HOST_PARAMS_MAX_BATCH + 1, 5000, 0, 0);
        k.options = KLSAMPLE_OPT_HOST_PARAMS;
        expect_error(&k, KLSAMPLE_ERR_INVALID_ARGUMENT);
        k.options = 0;
        CHECK(klsample_run(&k, nullptr) == KLSAMPLE_OK && stub::last_args.inline_flags == 0);
        // history_append needs history pairs and their ranges
        k.history_append = b.ids.data();
        expect_error(&k, KLSAMPLE_ERR_INVALID_ARGUMENT);
        k.options = KLSAMPLE_OPT_HISTORY_PAIRS;
        k.history_offsets = nullptr;
        expect_error(&k, KLSAMPLE_ERR_INVALID_ARGUMENT);
    }

    // the LM-head call: chunks of 1,024, one workgroup per chunk writes its histograms,
    // the logits are the output; argument errors before any launch
    {
        Bufs b;
        const int B = 5, V = 70001, N = 3, K = 50, d = 64;
        klsample_batch k = make_batch(b, B, V, N, K);
        size_t need = 0;
        CHECK(klsample_lmhead_workspace_size(B, V, K, N, &need) == KLSAMPLE_OK);
        b.ws.assign(need + 256, 0);
        k.workspace = (void *)(((uintptr_t)b.ws.data() + 255) & ~(uintptr_t)255);
        k.workspace_bytes = need;
        alignas(16) static uint16_t hid[B * d], wt[V * d / 1000 + 64];
        klsample_lmhead h = {hid, wt, d, 0};
        const int before = stub::launches;
        CHECK(klsample_lmhead_run(&k, &h, nullptr) == KLSAMPLE_OK && stub::launches == before + 1);
        check_plan(b, k, true);
        CHECK(stub::last_args.E == 4 && stub::last_args.C == 1024 && stub::last_args.wide_split == 0);
        CHECK(stub::last_head.dim == d && stub::last_head.logits_out == (const float *)k.logits);
        CHECK(klsample_lmhead_run(&k, nullptr, nullptr) == KLSAMPLE_ERR_INVALID_ARGUMENT);
        klsample_lmhead e = h; e.dim = 48;
        CHECK(klsample_lmhead_run(&k, &e, nullptr) == KLSAMPLE_ERR_INVALID_ARGUMENT);
        e = h; e.weight = (const unsigned char *)wt + 2;
        CHECK(klsample_lmhead_run(&k, &e, nullptr) == KLSAMPLE_ERR_INVALID_ARGUMENT);
        e = h; e.hidden = nullptr;
        CHECK(klsample_lmhead_run(&k, &e, nullptr) == KLSAMPLE_ERR_INVALID_ARGUMENT);
        klsample_batch kb = k; kb.dtype = KLSAMPLE_BFLOAT16;
        CHECK(klsample_lmhead_run(&kb, &h, nullptr) == KLSAMPLE_ERR_INVALID_ARGUMENT);
        kb = k; kb.row_stride = V + 4;
        CHECK(klsample_lmhead_run(&kb, &h, nullptr) == KLSAMPLE_ERR_INVALID_ARGUMENT);
        kb = k; kb.workspace_bytes = need - 1;
        CHECK(klsample_lmhead_run(&kb, &h, nullptr) == KLSAMPLE_ERR_WORKSPACE);
        CHECK(stub::launches == before + 1);
    }

    // workspace init and phase events
    {
        unsigned char buf[64];
        CHECK(klsample_workspace_init(nullptr, 10, nullptr) == KLSAMPLE_ERR_INVALID_ARGUMENT);
        CHECK(klsample_workspace_init(buf, 0, nullptr) == KLSAMPLE_OK);
        CHECK(klsample_workspace_init(buf, sizeof buf, nullptr) == KLSAMPLE_OK && stub::fills == 1);
        void *evs[4] = {nullptr, nullptr, nullptr, nullptr};
        CHECK(klsample_set_phase_events(evs, 5) == KLSAMPLE_ERR_INVALID_ARGUMENT);
        CHECK(klsample_set_phase_events(nullptr, 2) == KLSAMPLE_ERR_INVALID_ARGUMENT);
        CHECK(klsample_set_phase_events(evs, 4) == KLSAMPLE_OK);
        CHECK(klsample_set_phase_events(nullptr, 0) == KLSAMPLE_OK);
    }

    // the error string is per thread
    {
        std::string other;
        std::thread t([&] {
            klsample_batch *none = nullptr;
            klsample_run(none, nullptr);
            other = klsample_last_error();
        });
        t.join();
        size_t sz = 0;
        CHECK(klsample_workspace_size(1, 10, KLSAMPLE_FLOAT32, 0, 0, &sz) == KLSAMPLE_OK);
        CHECK(!other.empty() && strlen(klsample_last_error()) == 0);
    }

    if (failures) {
        fprintf(stderr, "%d checks failed\n", failures);
        return 1;
    }
    printf("ok\n");
    return 0;
}
