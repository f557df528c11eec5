// seoul_gpu.hpp — imi's engine API (imi/core/seoul.h:19-94, imi/brain.h:20-65), file API (imi/model.h:12-36), voice
// generator API (imi/core/voice.h:17-51), codec API (imi/core/codec.h:17-65) and ears API (imi/core/ears.h:17-51)
// over libseoul_hip's C ABI.
//
// Drop-in for the CPU engine: the same members and signatures, so imi's callers (greedy loops, the voice frame,
// step2 riding) compile unchanged after
//     #include "seoul_gpu.hpp"
//     using seoul_hip::imi_seoul; using seoul_hip::imi_seoul_state; using seoul_hip::imi_voice;
//     using seoul_hip::imi_brain; using seoul_hip::imi_file; using seoul_hip::imi_tensor; using seoul_hip::imi_codec;
//     using seoul_hip::imi_ears;
// and link -lseoul_hip. Header-only C++17; no HIP or torch types. The thread arguments of load() are accepted and
// ignored (the device has no thread team). Errors follow imi: load() returns false and prints; a full context
// prints "context full" and returns without stepping (imi/core/seoul.cpp:209,353,498).
#pragma once
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <map>
#include <string>
#include <utility>
#include <vector>

#include "seoul_hip.h"

namespace seoul_hip {

// The ggml_tensor fields imi's callers read (ggml is not part of this build): type, ne, nb, data, name.
struct imi_tensor {
    int type = 0;                     // ggml type id: 0 F32, 1 F16, 2 Q4_0, 3 Q4_1, 8 Q8_0, 14 Q6_K
    int64_t ne[4] = {1, 1, 1, 1};     // ne[0] innermost
    size_t nb[4] = {0, 0, 0, 0};      // ggml byte strides: nb[0] one element or block, nb[1] one row
    void* data = nullptr;             // host bytes; null once drop_data let the file go and the tensor was not kept
    char name[64] = {};               // ggml's name length
};
inline size_t imi_nbytes(const imi_tensor* t) { return t->nb[3] * (size_t)t->ne[3]; }   // ggml_nbytes

// imi_file (imi/model.h:12-36): one GGUF file read into host memory, tensors looked up by name. get() of a missing
// required tensor and a failed keep() print and exit, as imi does (imi/model.cpp:108-150). A tensor pointer stays
// valid as long as the file object; keep() and drop_data() update the data of pointers already handed out, as
// they update ggml's tensor headers in imi.
struct imi_file {
    void* data = nullptr;   // every tensor's bytes, one block (null after drop_data)
    size_t size = 0;

    imi_file() = default;
    imi_file(const imi_file&) = delete;
    imi_file& operator=(const imi_file&) = delete;
    ~imi_file() {
        if (h) sh_file_free(h);
    }

    // imi/model.cpp:48-106; `repack` (a CPU kernel layout) has no meaning here: the engine makes the device layout
    bool load(const std::string& path, bool repack = false) {
        (void)repack;
        if (h) sh_file_free(h);
        h = nullptr;
        cache.clear();
        data = nullptr;
        size = 0;
        if (sh_file_load(path.c_str(), &h) != SH_OK) {
            fprintf(stderr, "imi: %s\n", sh_last_error());
            return false;
        }
        const void* d = nullptr;
        sh_file_block(h, &d, &size);
        data = const_cast<void*>(d);
        return true;
    }
    imi_tensor* get(const std::string& name, bool required = true) const {
        sh_tensor t{};
        if (!h || sh_file_get(h, name.c_str(), &t) != SH_OK) return missing(name, required);
        return put(t);
    }
    int64_t key_i(const std::string& name, int64_t def) const { return h ? sh_file_key_i(h, name.c_str(), def) : def; }
    float key_f(const std::string& name, float def) const { return h ? sh_file_key_f(h, name.c_str(), def) : def; }
    // a copy of the tensor's bytes of its own (64-byte aligned), which drop_data() leaves in place
    imi_tensor* keep(const std::string& name, bool required = true) {
        sh_tensor t{};
        if (!h || sh_file_get(h, name.c_str(), &t) != SH_OK) return missing(name, required);
        if (sh_file_keep(h, name.c_str(), &t) != SH_OK) {
            fprintf(stderr, "imi: out of memory keeping %s\n", name.c_str());
            exit(1);
        }
        return put(t);
    }
    void drop_data() {
        if (!h || !data) return;
        sh_file_drop_data(h);
        for (auto& e : cache) {
            sh_tensor t{};
            if (sh_file_get(h, e.first.c_str(), &t) == SH_OK) e.second.data = t.data;
        }
        data = nullptr;
        size = 0;
    }
    // the integers or bools of an array key (imi reads these through the file's gguf context): empty when absent
    std::vector<int64_t> key_arr(const std::string& name) const {
        std::vector<int64_t> v;
        const int n = h ? sh_file_key_arr(h, name.c_str(), nullptr, 0) : 0;
        if (n > 0) {
            v.resize((size_t)n);
            sh_file_key_arr(h, name.c_str(), v.data(), n);
        }
        return v;
    }

private:
    sh_file* h = nullptr;
    mutable std::map<std::string, imi_tensor> cache;   // stable addresses, one header per tensor as in ggml
    imi_tensor* put(const sh_tensor& t) const {
        imi_tensor& e = cache[t.name];
        e.type = t.type;
        for (int d = 0; d < 4; d++) {
            e.ne[d] = t.ne[d];
            e.nb[d] = t.nb[d];
        }
        e.data = t.data;
        snprintf(e.name, sizeof e.name, "%s", t.name);
        return &e;
    }
    static imi_tensor* missing(const std::string& name, bool required) {
        if (required) {
            fprintf(stderr, "imi: missing tensor %s\n", name.c_str());
            exit(1);
        }
        return nullptr;
    }
};

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
    // the model file: keys and tensor shapes readable; the norm vectors kept on the host as imi keeps them
    // (imi/core/seoul.cpp:94-165), every table's bytes let go once they are on the device
    imi_file f;
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
        if (!f.load(path)) return false;
        sh_model_info I{};
        sh_info(ctx, &I);
        n_embd = I.n_embd; n_vocab = I.n_vocab; n_head = I.n_head; n_head_kv = I.n_head_kv; head_dim = I.head_dim;
        n_ff = I.n_ff; d_conv = I.d_conv; n_swa = I.n_swa; n_ctx = I.n_ctx;
        f.keep("output_norm.weight");
        f.keep("rope_freqs.weight", false);
        for (int il = 0; il < I.n_layer; il++) {
            const std::string p = "blk." + std::to_string(il) + ".";
            for (const char* n : {"attn_norm.weight", "post_attention_norm.weight", "ffn_norm.weight", "post_ffw_norm.weight"})
                f.keep(p + n);
            if (f.get(p + "attn_q_norm.weight", false)) {
                f.keep(p + "attn_q_norm.weight");
                f.keep(p + "attn_k_norm.weight");
            }
        }
        f.drop_data();
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

// imi_brain (imi/brain.h:20-65): the same model through imi's ggml-graph engine interface. The layer tensors are the
// file's (shapes and, as the file stays loaded, bytes readable); the step runs on the device engine, whose numbers
// follow imi_seoul's op order (imi/core/seoul.cpp:352-488). The CPU engine's own members (ggml contexts, thread pool,
// arenas, repacked tables, per-step call lists) have no counterpart: the K/V caches and conv memory are device
// memory of the engine's state. The stacked q|k|v|gate and gate|up tables exist only in the device layout, so
// qkvg and gate_up stay null. `n_threads` is kept and ignored.
struct imi_brain {
    struct layer {
        imi_tensor *attn_norm = nullptr, *post_attn_norm = nullptr, *ffn_norm = nullptr, *post_ffn_norm = nullptr;
        imi_tensor *ffn_up = nullptr, *ffn_gate = nullptr, *ffn_down = nullptr;
        // short conv
        imi_tensor *conv_w = nullptr, *in_proj = nullptr, *out_proj = nullptr;
        // attention
        imi_tensor *q = nullptr, *k = nullptr, *v = nullptr, *o = nullptr, *gate = nullptr, *q_norm = nullptr, *k_norm = nullptr;
        bool swa = false;
        imi_tensor *qkvg = nullptr, *gate_up = nullptr;
        int attn_index = -1;
    };

    imi_file f;
    imi_tensor *tok_embd = nullptr, *out_norm = nullptr, *rope_freqs = nullptr;
    std::vector<layer> layers;
    int n_embd = 0, n_vocab = 0, n_head = 0, n_head_kv = 0, head_dim = 0, d_conv = 0, n_swa = 0, n_ctx = 0;
    float eps = 1e-5f, rope_base = 1e6f, rope_base_swa = 1e4f;
    int pos = 0;
    int n_threads = 4;
    std::vector<float> hidden, logits;

    imi_brain() = default;
    imi_brain(const imi_brain&) = delete;
    imi_brain& operator=(const imi_brain&) = delete;
    ~imi_brain() {
        if (st) sh_state_free(st);
        if (ctx) sh_destroy(ctx);
    }

    // imi/brain.cpp:11-82: the file's keys and tensors, then the model on the device with a context of ctx_len
    bool load(const std::string& path, int threads, int ctx_len, int device = 0) {
        n_threads = threads;
        if (!f.load(path)) return false;
        tok_embd = f.get("token_embd.weight");
        out_norm = f.get("output_norm.weight");
        rope_freqs = f.get("rope_freqs.weight", false);
        n_embd = (int)tok_embd->ne[0];
        n_vocab = (int)tok_embd->ne[1];
        eps = f.key_f("lfm3.attention.layer_norm_rms_epsilon", 1e-5f);
        rope_base = f.key_f("lfm3.rope.freq_base", 1e6f);
        rope_base_swa = f.key_f("lfm3.rope.freq_base_swa", 1e4f);
        n_swa = (int)f.key_i("lfm3.attention.sliding_window", 0);
        d_conv = (int)f.key_i("lfm3.shortconv.l_cache", 7) - 1;
        n_head = (int)f.key_i("lfm3.attention.head_count", 16);
        head_dim = (int)f.key_i("lfm3.attention.key_length", 128);
        const int n_layer = (int)f.key_i("lfm3.block_count", 0);
        const std::vector<int64_t> swa = f.key_arr("lfm3.attention.sliding_window_pattern");
        layers.clear();
        int n_attn = 0;
        for (int il = 0; il < n_layer; il++) {
            const std::string p = "blk." + std::to_string(il) + ".";
            layer L;
            L.attn_norm = f.get(p + "attn_norm.weight");
            L.post_attn_norm = f.get(p + "post_attention_norm.weight");
            L.ffn_norm = f.get(p + "ffn_norm.weight");
            L.post_ffn_norm = f.get(p + "post_ffw_norm.weight");
            L.ffn_up = f.get(p + "ffn_up.weight");
            L.ffn_gate = f.get(p + "ffn_gate.weight");
            L.ffn_down = f.get(p + "ffn_down.weight");
            if (f.get(p + "shortconv.conv.weight", false)) {
                L.conv_w = f.get(p + "shortconv.conv.weight");
                L.in_proj = f.get(p + "shortconv.in_proj.weight");
                L.out_proj = f.get(p + "shortconv.out_proj.weight");
            } else {
                L.q = f.get(p + "attn_q.weight");
                L.k = f.get(p + "attn_k.weight");
                L.v = f.get(p + "attn_v.weight");
                L.o = f.get(p + "attn_output.weight");
                L.gate = f.get(p + "attn_gate.weight");
                L.q_norm = f.get(p + "attn_q_norm.weight");
                L.k_norm = f.get(p + "attn_k_norm.weight");
                L.swa = il < (int)swa.size() && swa[(size_t)il] != 0;
                L.attn_index = n_attn++;
                n_head_kv = (int)(L.k->ne[1] / head_dim);
            }
            layers.push_back(L);
        }
        n_ctx = ctx_len;
        if (sh_create(device, &ctx) != SH_OK || sh_load(ctx, path.c_str(), ctx_len) != SH_OK || sh_state_new(ctx, &st) != SH_OK) {
            fprintf(stderr, "seoul-hip: load: %s\n", sh_last_error());
            return false;
        }
        hidden.assign(n_embd, 0.0f);
        logits.assign(n_vocab, 0.0f);
        pos = 0;
        return true;
    }
    // imi/brain.cpp:144-147: back to position 0, conv memory cleared
    void reset() {
        sh_state_reset(st);
        pos = 0;
    }
    // one step (imi/brain.cpp:149-288): a word (token >= 0) or a ready input vector; hidden always, logits when asked
    void step(int32_t token, const float* embd, bool want_logits) {
        int cur = -1;
        sh_state_pos(st, &cur);
        if (cur != pos) sh_state_set_pos(st, pos);
        int32_t best = -1;
        if (sh_step(ctx, st, token, embd, want_logits, hidden.data(), want_logits ? logits.data() : nullptr, &best) == SH_OK) pos++;
        else fprintf(stderr, "seoul-hip: step: %s\n", sh_last_error());
    }

private:
    sh_ctx* ctx = nullptr;
    sh_state* st = nullptr;
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

// imi_codec (imi/core/codec.h:17-65) over the same C ABI: the codec decoder on the device. frame() appends the
// frame's samples to pcm (1920, less the start padding after a reset), flush() the tail the overlap holds back.
// `threads` and `shared` (CPU thread team) are accepted and ignored.
struct imi_codec {
    int n_lvl = 0, n_cb = 12, n_embd = 0, n_ff = 0, n_head = 0, n_head_kv = 0, head_dim = 0, d_conv = 0;
    int n_fs = 6, window = 30, n_fft = 1280, hop = 320, n_bins = 641;
    float eps = 1e-5f, theta = 1e6f;
    int n_threads = 4;

    imi_codec() = default;
    imi_codec(const imi_codec&) = delete;
    imi_codec& operator=(const imi_codec&) = delete;
    ~imi_codec() {
        if (c) sh_codec_free(c);
    }

    bool load(const std::string& path, int threads, void* shared = nullptr, int device = 0) {   // codec.cpp:41-108
        (void)shared;
        n_threads = threads;
        if (sh_codec_load(device, path.c_str(), &c) != SH_OK) return report("load");
        sh_codec_shape I{};
        sh_codec_info(c, &I);
        n_lvl = I.n_lvl; n_embd = I.n_embd; n_ff = I.n_ff; n_head = I.n_head; n_head_kv = I.n_head_kv;
        head_dim = I.head_dim; d_conv = I.d_conv; n_bins = I.n_bins;
        return true;
    }
    void reset() {   // codec.cpp:110-119
        if (sh_codec_reset(c) != SH_OK) report("reset");
    }
    void frame(const int32_t* codes, std::vector<float>& pcm) {   // codec.cpp:121-127
        float buf[1920];
        int n = 0;
        if (sh_codec_frame(c, codes, buf, &n) != SH_OK) { report("frame"); return; }
        pcm.insert(pcm.end(), buf, buf + n);
    }
    void flush(std::vector<float>& pcm) {   // codec.cpp:271-277
        float buf[1280];
        int n = 0;
        if (sh_codec_flush(c, buf, &n) != SH_OK) { report("flush"); return; }
        pcm.insert(pcm.end(), buf, buf + n);
    }

private:
    sh_codec* c = nullptr;
    bool report(const char* what) const {
        fprintf(stderr, "seoul-hip: codec %s: %s\n", what, sh_last_error());
        return false;
    }
};

// imi_ears (imi/core/ears.h:17-51) over the same C ABI: the audio encoder on the device. encode() turns 16 kHz samples
// from the clip's start into [n_pos][n_out] rows for the brain's step_batch and returns n_pos; last_mel holds the
// encode's [n_frames][n_mel] log-mel frames. `threads` and `shared` (CPU thread team) are accepted and ignored; the
// stage timers stay 0 (the whole encode is one device call).
struct imi_ears {
    int n_mel = 128, n_bin = 201, n_fft = 400, hop = 160, n_ch = 256, n_embd = 768, n_ff = 0, n_head = 0, n_head_kv = 0,
        head_dim = 0, window = 32, n_out = 0, d_conv = 3;
    float eps = 1e-5f, rope_theta = 1e6f;
    int n_threads = 4;
    double t_mel = 0, t_down = 0, t_layers = 0, t_proj = 0;
    std::vector<float> last_mel;

    imi_ears() = default;
    imi_ears(const imi_ears&) = delete;
    imi_ears& operator=(const imi_ears&) = delete;
    ~imi_ears() {
        if (e) sh_ears_free(e);
    }

    bool load(const std::string& path, int threads, void* shared = nullptr, int device = 0) {   // ears.cpp:40-138
        (void)shared;
        n_threads = threads;
        if (sh_ears_load(device, path.c_str(), &e) != SH_OK) return report("load");
        sh_ears_shape I{};
        sh_ears_info(e, &I);
        n_mel = I.n_mel; n_ch = I.n_ch; n_embd = I.n_embd; n_ff = I.n_ff; n_head = I.n_head; n_head_kv = I.n_head_kv;
        head_dim = I.head_dim; window = I.window; n_out = I.n_out; d_conv = I.d_conv;
        return true;
    }
    int encode(const float* pcm, int n, std::vector<float>& out) {   // ears.cpp:198-407
        int P = 0, F = 0;
        if (sh_ears_positions(e, n, &P, &F) != SH_OK) return report("encode"), 0;
        out.resize((size_t)P * n_out);
        if (sh_ears_encode(e, pcm, n, out.data(), &P) != SH_OK) return report("encode"), 0;
        last_mel.resize((size_t)F * n_mel);
        if (sh_ears_mel(e, last_mel.data(), F, &F) != SH_OK) report("mel");
        return P;
    }

private:
    sh_ears* e = nullptr;
    bool report(const char* what) const {
        fprintf(stderr, "seoul-hip: ears %s: %s\n", what, sh_last_error());
        return false;
    }
};

}  // namespace seoul_hip
