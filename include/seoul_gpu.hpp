// seoul_gpu.hpp — imi's engine API (imi/core/seoul.h:19-94, imi/brain.h:20-65) and voice generator API
// (imi/core/voice.h:17-51) over libseoul_hip's C ABI.
//
// Drop-in for the CPU engine: the same members and signatures, so imi's callers (greedy loops, the voice frame,
// step2 riding) compile unchanged after
//     #include "seoul_gpu.hpp"
//     using seoul_hip::imi_seoul; using seoul_hip::imi_seoul_state; using seoul_hip::imi_voice;
// and link -lseoul_hip. Header-only C++17; no HIP or torch types. The thread arguments of load() are accepted and
// ignored (the device has no thread team). Errors follow imi: load() returns false and prints; a full context
// prints "context full" and returns without stepping (imi/core/seoul.cpp:209,353,498).
#pragma once
#include <cstdint>
#include <cstdio>
#include <string>
#include <utility>
#include <vector>

#include "seoul_hip.h"

namespace seoul_hip {

// one conversation's memory and latest outputs (imi/core/seoul.h:21-26); the K/V caches and conv memory live on the
// device, owned by the handle
struct imi_seoul_state {
    int pos = 0;
    std::vector<float> hidden, logits;
    sh_state* handle = nullptr;

    imi_seoul_state() = default;
    imi_seoul_state(const imi_seoul_state&) = delete;
    imi_seoul_state& operator=(const imi_seoul_state&) = delete;
    imi_seoul_state(imi_seoul_state&& o) noexcept { *this = std::move(o); }
    imi_seoul_state& operator=(imi_seoul_state&& o) noexcept {
        if (this != &o) {
            release();
            pos = o.pos;
            hidden = std::move(o.hidden);
            logits = std::move(o.logits);
            handle = o.handle;
            o.handle = nullptr;
        }
        return *this;
    }
    ~imi_seoul_state() { release(); }
    void release() {
        if (handle) sh_state_free(handle);
        handle = nullptr;
    }
};

struct imi_seoul {
    int n_embd = 0, n_vocab = 0, n_head = 0, n_head_kv = 0, head_dim = 0, n_ff = 0, d_conv = 0, n_swa = 0, n_ctx = 0;
    int n_threads = 1;
    // the brain's own conversation, as in imi (pos may be set back to rewind, imi/core/hear_pieces.cpp:8-11)
    int pos = 0;
    std::vector<float> hidden, logits;

    imi_seoul() = default;
    imi_seoul(const imi_seoul&) = delete;
    imi_seoul& operator=(const imi_seoul&) = delete;
    ~imi_seoul() {
        own.release();
        if (ctx) sh_destroy(ctx);
    }

    // imi/core/seoul.cpp:93-186; `shared` (a CPU thread team) has no meaning here and is ignored
    bool load(const std::string& path, int threads, int ctx_len, void* shared = nullptr, int device = 0) {
        (void)threads;
        (void)shared;
        if (sh_create(device, &ctx) != SH_OK || sh_load(ctx, path.c_str(), ctx_len) != SH_OK) return report("load");
        sh_model_info I{};
        sh_info(ctx, &I);
        n_embd = I.n_embd; n_vocab = I.n_vocab; n_head = I.n_head; n_head_kv = I.n_head_kv; head_dim = I.head_dim;
        n_ff = I.n_ff; d_conv = I.d_conv; n_swa = I.n_swa; n_ctx = I.n_ctx;
        own = new_state();
        hidden.assign(n_embd, 0.0f);
        logits.assign(n_vocab, 0.0f);
        return own.handle != nullptr;
    }
    void reset() {   // imi/core/seoul.cpp:188-191
        sh_state_reset(own.handle);
        pos = 0;
    }
    void step(int32_t token, const float* embd, bool want_logits) {   // seoul.cpp:352-357
        sync_pos(own, pos);
        int32_t best = -1;
        if (sh_step(ctx, own.handle, token, embd, want_logits, hidden.data(), want_logits ? logits.data() : nullptr, &best) == SH_OK) pos++;
        else report("step");
    }
    // tokens[n] or embd[n][n_embd]; hidden (and logits) of the last position, every hidden in hidden_all
    void step_batch(const int32_t* tokens, const float* embd, int n, bool want_logits, float* hidden_all = nullptr) {
        sync_pos(own, pos);
        int32_t best = -1;
        if (sh_step_batch(ctx, own.handle, tokens, embd, n, want_logits, hidden.data(), want_logits ? logits.data() : nullptr,
                          hidden_all, &best) == SH_OK)
            pos += n;
        else report("step_batch");
    }
    imi_seoul_state new_state() const {   // seoul.cpp:193-201
        imi_seoul_state s;
        if (sh_state_new(ctx, &s.handle) != SH_OK) report("new_state");
        s.hidden.assign(n_embd, 0.0f);
        s.logits.assign(n_vocab, 0.0f);
        return s;
    }
    void swap_state(imi_seoul_state& s) {   // seoul.cpp:203-206: O(1)
        own.pos = pos;
        own.hidden.swap(hidden);
        own.logits.swap(logits);
        std::swap(own.pos, s.pos);
        std::swap(own.handle, s.handle);
        own.hidden.swap(s.hidden);
        own.logits.swap(s.logits);
        pos = own.pos;
        hidden.swap(own.hidden);
        logits.swap(own.logits);
    }
    // two conversations, one read of every table (seoul.cpp:208-220)
    void step2(int32_t token_a, const float* embd_a, bool logits_a, imi_seoul_state& b, int32_t token_b, const float* embd_b,
               bool logits_b) {
        sync_pos(own, pos);
        sync_pos(b, b.pos);
        int32_t ba = -1, bb = -1;
        if (sh_step2(ctx, own.handle, token_a, embd_a, logits_a, b.handle, token_b, embd_b, logits_b, hidden.data(),
                     logits_a ? logits.data() : nullptr, &ba, b.hidden.data(), logits_b ? b.logits.data() : nullptr, &bb) == SH_OK) {
            pos++;
            b.pos++;
        } else {
            report("step2");
        }
    }
    // every layer table read back to back, ncol inputs riding each read; best ms over reps (seoul.cpp:657-685)
    double bench_tables(int ncol, int reps) {
        double ms = 0, us = 0, bytes = 0;
        int n = 0;
        if (sh_bench_tables(ctx, ncol, reps, &ms, &us, &bytes, &n) != SH_OK) report("bench_tables");
        return ms;
    }

private:
    sh_ctx* ctx = nullptr;
    imi_seoul_state own;
    void sync_pos(imi_seoul_state& s, int p) const {
        int cur = -1;
        sh_state_pos(s.handle, &cur);
        if (cur != p) sh_state_set_pos(s.handle, p);
        s.pos = p;
    }
    bool report(const char* what) const {
        fprintf(stderr, "seoul-hip: %s: %s\n", what, sh_last_error());
        return false;
    }
};

// imi_voice (imi/core/voice.h:17-51) over the same C ABI: the Q8_0 voice generator on the device. `base` is the
// frame's projected input, refreshed by begin_frame as in imi.
struct imi_voice {
    int n_embd = 0, n_vocab = 0, n_cb = 0, n_in = 0, n_head = 0, n_head_kv = 0, head_dim = 0, n_ff = 0;
    float eps = 1e-5f, rope_theta = 1e6f;
    int n_threads = 4;
    std::vector<float> base;   // [n_cb][n_embd]

    imi_voice() = default;
    imi_voice(const imi_voice&) = delete;
    imi_voice& operator=(const imi_voice&) = delete;
    ~imi_voice() {
        if (v) sh_voice_free(v);
    }

    // imi/core/voice.cpp:27-88; `threads` and `shared` (CPU thread team) are ignored on the device
    bool load(const std::string& path, int threads, void* shared = nullptr, int device = 0) {
        (void)shared;
        n_threads = threads;
        if (sh_voice_load(device, path.c_str(), &v) != SH_OK) return report("load");
        sh_voice_shape I{};
        sh_voice_info(v, &I);
        n_embd = I.n_embd; n_vocab = I.n_vocab; n_cb = I.n_cb; n_in = I.n_in; n_head = I.n_head;
        n_head_kv = I.n_head_kv; head_dim = I.head_dim; n_ff = I.n_ff;
        base.assign((size_t)n_cb * n_embd, 0.0f);
        return true;
    }
    void begin_frame(const float* h) {   // voice.cpp:99-111
        if (sh_voice_begin_frame(v, h) != SH_OK || sh_voice_base(v, base.data()) != SH_OK) report("begin_frame");
    }
    // the brain's next input after a frame: the sum of the codes' feedback rows, n_in wide (voice.cpp:90-97)
    void feedback(const int32_t* codes, float* out) const {
        if (sh_voice_feedback(v, codes, out) != SH_OK) report("feedback");
    }
    // codes[i] < 0 = still masked; scores of the codebooks in `need`, [need.size()][n_vocab] (voice.cpp:113-117)
    void pass(const int32_t* codes, const std::vector<int>& need, std::vector<float>& out) {
        out.resize(need.size() * (size_t)n_vocab);
        std::vector<int32_t> nd(need.begin(), need.end());
        if (sh_voice_pass(v, codes, nd.data(), (int)nd.size(), out.data()) != SH_OK) report("pass");
    }
    // imi_talker::next's picks for the codebooks the last pass scored (imi/core/talk.cpp:147-164), on the device:
    // hist = the last n_frames frames of codes (n_cb each), u = one uniform draw in [0, 1) per pick, drawn by the
    // caller from its generator; keep[j] = 1 - p[end-of-audio] / sum. The scores `pass` returned are not changed.
    bool sample(const int32_t* hist, int n_frames, const double* u, float temp, float rep, int32_t* picks,
                double* keep) {
        if (sh_voice_sample(v, hist, n_frames, u, temp, rep, picks, keep) != SH_OK) return report("sample");
        return true;
    }

private:
    sh_voice* v = nullptr;
    bool report(const char* what) const {
        fprintf(stderr, "seoul-hip: voice %s: %s\n", what, sh_last_error());
        return false;
    }
};

}  // namespace seoul_hip
