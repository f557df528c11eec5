// ORACLE — test infrastructure only (see imi_cpu.h). Engine-level restatement of imi's brain step
// (imi/core/seoul.cpp) and voice generator (imi/core/voice.cpp), with a thread team shaped like imi_team
// (imi/core/team.h) so that, timed, it stands for imi's CPU path.
#include "imi_cpu.h"

#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <algorithm>
#include <atomic>
#include <chrono>
#include <cmath>
#include <cstdio>
#include <cstring>
#include <functional>
#include <immintrin.h>
#include <memory>
#include <thread>

namespace orc {

// ---------------------------------------------------------------- GGUF v3 reader (own code)
namespace {
struct rd {
    const uint8_t* p; size_t n, o = 0; bool bad = false;
    template <class T> T get() { T v{}; if (o + sizeof(T) > n) { bad = true; return v; } memcpy(&v, p + o, sizeof(T)); o += sizeof(T); return v; }
    std::string str() { uint64_t l = get<uint64_t>(); if (bad || o + l > n) { bad = true; return {}; } std::string s((const char*)p + o, l); o += l; return s; }
};
size_t type_size(int t, int64_t ne0, size_t* row) {   // bytes of one row of ne0 values
    size_t r = 0;
    switch (t) {
        case T_F32: r = 4 * ne0; break;
        case T_F16: r = 2 * ne0; break;
        case T_Q4_0: r = ne0 / 32 * 18; break;
        case T_Q4_1: r = ne0 / 32 * 20; break;
        case T_Q8_0: r = ne0 / 32 * 34; break;
        case T_Q6_K: r = ne0 / 256 * 210; break;
        default: return 0;
    }
    *row = r;
    return r;
}
}  // namespace

bool gfile::open(const std::string& path) {
    const int fd = ::open(path.c_str(), O_RDONLY);
    if (fd < 0) { fprintf(stderr, "oracle: cannot open %s\n", path.c_str()); return false; }
    struct stat st;
    fstat(fd, &st);
    map_size = (size_t)st.st_size;
    map = mmap(nullptr, map_size, PROT_READ, MAP_PRIVATE, fd, 0);
    ::close(fd);
    if (map == MAP_FAILED) { map = nullptr; return false; }
    rd r{(const uint8_t*)map, map_size};
    if (r.get<uint32_t>() != 0x46554747u) return false;   // "GGUF"
    const uint32_t ver = r.get<uint32_t>();
    if (ver < 2) return false;
    const uint64_t nt = r.get<uint64_t>(), nkv = r.get<uint64_t>();
    size_t align = 32;
    auto read_scalar = [&](int t, kv& k) {
        switch (t) {
            case 0: k.i = r.get<uint8_t>(); break;  case 1: k.i = r.get<int8_t>(); break;
            case 2: k.i = r.get<uint16_t>(); break; case 3: k.i = r.get<int16_t>(); break;
            case 4: k.i = r.get<uint32_t>(); break; case 5: k.i = r.get<int32_t>(); break;
            case 6: k.f = r.get<float>(); k.i = (int64_t)k.f; break;
            case 7: k.i = r.get<uint8_t>(); break;
            case 8: r.str(); break;
            case 10: k.i = (int64_t)r.get<uint64_t>(); break; case 11: k.i = r.get<int64_t>(); break;
            case 12: k.f = r.get<double>(); k.i = (int64_t)k.f; break;
            default: r.bad = true;
        }
        if (t != 6 && t != 12) k.f = (double)k.i;
    };
    for (uint64_t i = 0; i < nkv && !r.bad; i++) {
        kv k;
        k.key = r.str();
        k.type = (int)r.get<uint32_t>();
        k.i = 0; k.f = 0;
        if (k.type == 9) {
            const int et = (int)r.get<uint32_t>();
            const uint64_t cnt = r.get<uint64_t>();
            for (uint64_t e = 0; e < cnt && !r.bad; e++) { kv tmp; read_scalar(et, tmp); k.arr.push_back(tmp.i); }
        } else {
            read_scalar(k.type, k);
        }
        if (k.key == "general.alignment") align = (size_t)k.i;
        kvs.push_back(std::move(k));
    }
    for (uint64_t i = 0; i < nt && !r.bad; i++) {
        gtensor t;
        t.name = r.str();
        t.n_dims = (int)r.get<uint32_t>();
        for (int d = 0; d < t.n_dims && d < 4; d++) t.ne[d] = (int64_t)r.get<uint64_t>();
        t.type = (int)r.get<uint32_t>();
        t.offset = r.get<uint64_t>();
        size_t row = 0;
        if (!type_size(t.type, t.ne[0], &row)) { fprintf(stderr, "oracle: tensor %s has unsupported type %d\n", t.name.c_str(), t.type); return false; }
        t.row_bytes = row;
        t.nbytes = row * t.ne[1] * t.ne[2] * t.ne[3];
        tensors.push_back(std::move(t));
    }
    if (r.bad) return false;
    const size_t data0 = (r.o + align - 1) / align * align;
    for (auto& t : tensors) {
        if (data0 + t.offset + t.nbytes > map_size) { fprintf(stderr, "oracle: short file at %s\n", t.name.c_str()); return false; }
        t.data = (const uint8_t*)map + data0 + t.offset;
    }
    return true;
}
const gtensor* gfile::get(const std::string& name) const {
    for (auto& t : tensors) if (t.name == name) return &t;
    return nullptr;
}
int64_t gfile::key_i(const std::string& key, int64_t def) const {
    for (auto& k : kvs) if (k.key == key && k.type != 9) return k.i;
    return def;
}
float gfile::key_f(const std::string& key, float def) const {
    for (auto& k : kvs) if (k.key == key && k.type != 9) return (float)k.f;
    return def;
}
const std::vector<int64_t>* gfile::key_arr(const std::string& key) const {
    for (auto& k : kvs) if (k.key == key && k.type == 9) return &k.arr;
    return nullptr;
}
gfile::~gfile() { if (map) munmap(map, map_size); }


static inline float silu(float x) { return x / (1.0f + expf(-x)); }   // imi/core/seoul.cpp:48

// ---------------------------------------------------------------- brain engine (imi/core/seoul.{h,cpp})
struct state {   // imi_seoul_state (imi/core/seoul.h:21-26)
    std::vector<std::vector<uint16_t>> k_cache, v_cache;   // per attention layer [n_ctx][kvd]
    std::vector<std::vector<float>> conv_state;            // per layer [d_conv][E], oldest first
    int pos = 0;
    std::vector<float> hidden, logits;
};

struct engine {
    struct layer {
        const float *attn_norm = nullptr, *post_attn_norm = nullptr, *ffn_norm = nullptr, *post_ffn_norm = nullptr;
        const float *q_norm = nullptr, *k_norm = nullptr;
        std::vector<float> conv_w;   // [tap][channel]
        q4tab in_proj, out_proj, qkvg, o, gate_up, down;
        bool conv = false, swa = false;
        int ai = -1;
    };
    gfile f;
    std::vector<layer> layers;
    q4tab vocab;                     // tied Q4_0 word table in the 8-row layout (word scores)
    bool vocab_q6k = false;          // the word table is Q6_K (imi's own format): read as stored, rows of 210-byte blocks
    const gtensor* tok = nullptr;    // tied word table as stored (input rows)
    const float *out_norm = nullptr, *rope_freqs = nullptr;
    int n_embd = 0, n_vocab = 0, n_head = 0, n_head_kv = 0, head_dim = 0, n_ff = 0, d_conv = 0, n_swa = 0, n_ctx = 0;
    float eps = 1e-5f, rope_base = 1e6f, rope_base_swa = 1e4f;
    state own;
    team tm;
    int n_threads = 1;
    struct per_thread { std::vector<float> x, h, t, u, x2; q8in qi, qi2; q8kin qk; };
    std::vector<per_thread> per;
    std::vector<float> bcx, qkv, att, y, act, fo, bcx2, qkv2, att2, y2, act2, fo2;
    std::unique_ptr<std::atomic<int>[]> ctr;
    static constexpr int n_ctr = 512;
    static constexpr int NB = 64;
    std::vector<float> bX, bH, bBig, bY, bAct;
    q8b bq;
    // the int8 codes of every input cut a single step makes, in the order it makes them (thread 0's copy: every
    // thread cuts the same input alike), kept while trace_cuts is set; the float64 model takes them as its own cuts
    bool trace_cuts = false;
    std::vector<int8_t> cut_trace;

    bool load(const std::string& path, int threads, int ctx_len);
    void embed(int32_t token, const float* embd, float* x) const;
    void word_scores(per_thread& T, const float* hid, float* lg, std::atomic<int>& k);
    void reset_counters() { for (int i = 0; i < n_ctr; i++) ctr[i].store(0, std::memory_order_relaxed); }
    void step(int32_t token, const float* embd, bool want_logits);
    void step2(int32_t ta, const float* ea, bool la, state& b, int32_t tb, const float* eb, bool lb);
    void step_batch(const int32_t* tokens, const float* embd, int n, bool want_logits, float* hidden_all);
    state new_state() const;
    void run(int tid, int32_t token, const float* embd, bool want_logits);
    void run2(int tid, state& B, const int32_t tk[2], const float* const em[2], const bool want[2]);
    void run_batch(int tid, const int32_t* tokens, const float* embd, int n, float* hidden_all);
    void attend(const layer& L, const float* qkv_row, uint16_t* kc, uint16_t* vc, int p, int g, float* att_out, float* sc_buf) const;
};

static const float* f32(const gtensor* t) { return t ? (const float*)t->data : nullptr; }

// imi/core/seoul.cpp:93-186. The word table is Q6_K as imi requires (seoul.cpp:96), or Q4_0 (its rows repacked like
// any layer table and scored with the layer tables' kernel)
bool engine::load(const std::string& path, int threads, int ctx_len) {
    if (!f.open(path)) return false;
    tok = f.get("token_embd.weight");
    if (!tok || (tok->type != T_Q4_0 && tok->type != T_Q6_K)) { fprintf(stderr, "oracle: word table must be Q6_K or Q4_0\n"); return false; }
    vocab_q6k = tok->type == T_Q6_K;
    if (vocab_q6k && tok->ne[0] % 256) { fprintf(stderr, "oracle: Q6_K word table needs n_embd %% 256 == 0\n"); return false; }
    n_embd = (int)tok->ne[0]; n_vocab = (int)tok->ne[1];
    out_norm = f32(f.get("output_norm.weight"));
    rope_freqs = f32(f.get("rope_freqs.weight"));
    eps = f.key_f("lfm3.attention.layer_norm_rms_epsilon", 1e-5f);
    rope_base = f.key_f("lfm3.rope.freq_base", 1e6f);
    rope_base_swa = f.key_f("lfm3.rope.freq_base_swa", 1e4f);
    n_swa = (int)f.key_i("lfm3.attention.sliding_window", 0);
    d_conv = (int)f.key_i("lfm3.shortconv.l_cache", 7) - 1;
    n_head = (int)f.key_i("lfm3.attention.head_count", 16);
    head_dim = (int)f.key_i("lfm3.attention.key_length", 128);
    const int n_layer = (int)f.key_i("lfm3.block_count", 0);
    std::vector<bool> swa(n_layer, false);
    if (auto* a = f.key_arr("lfm3.attention.sliding_window_pattern"))
        for (int i = 0; i < n_layer && i < (int)a->size(); i++) swa[i] = (*a)[i] != 0;
    auto rows_of = [](std::vector<const uint8_t*>& o, const gtensor* t, int r0, int n) {
        for (int r = r0; r < r0 + n; r++) o.push_back(t->data + (size_t)r * t->row_bytes);
    };
    auto need = [&](const std::string& n) {
        const gtensor* t = f.get(n);
        if (!t) { fprintf(stderr, "oracle: missing tensor %s\n", n.c_str()); }
        return t;
    };
    // a table's stacked parts are all Q4_0 or all Q4_1 (imi/core/tables.cpp:70-72)
    auto whole = [&](q4tab& dst, std::vector<const gtensor*> parts) {
        std::vector<const uint8_t*> o;
        for (auto* p : parts) {
            if (!p || (p->type != T_Q4_0 && p->type != T_Q4_1) || p->type != parts[0]->type) return false;
            rows_of(o, p, 0, (int)p->ne[1]);
        }
        return q4_build(dst, o, (int)parts[0]->ne[0], parts[0]->type == T_Q4_1);
    };
    int n_attn = 0;
    layers.resize(n_layer);
    for (int il = 0; il < n_layer; il++) {
        const std::string p = "blk." + std::to_string(il) + ".";
        layer& L = layers[il];
        L.attn_norm = f32(need(p + "attn_norm.weight"));
        L.post_attn_norm = f32(need(p + "post_attention_norm.weight"));
        L.ffn_norm = f32(need(p + "ffn_norm.weight"));
        L.post_ffn_norm = f32(need(p + "post_ffw_norm.weight"));
        if (!L.attn_norm || !L.post_attn_norm || !L.ffn_norm || !L.post_ffn_norm) return false;
        bool ok = true;
        if (const gtensor* cw = f.get(p + "shortconv.conv.weight")) {
            L.conv = true;
            const int K = (int)cw->ne[0], C = (int)cw->ne[1];   // file [channel][tap] -> ours [tap][channel]
            L.conv_w.resize((size_t)K * C);
            for (int e = 0; e < C; e++) for (int k = 0; k < K; k++) L.conv_w[(size_t)k * C + e] = ((const float*)cw->data)[(size_t)e * K + k];
            ok &= whole(L.in_proj, {need(p + "shortconv.in_proj.weight")});
            ok &= whole(L.out_proj, {need(p + "shortconv.out_proj.weight")});
        } else {
            const gtensor* k = need(p + "attn_k.weight");
            ok &= whole(L.qkvg, {need(p + "attn_q.weight"), k, need(p + "attn_v.weight"), need(p + "attn_gate.weight")});
            ok &= whole(L.o, {need(p + "attn_output.weight")});
            L.q_norm = f32(need(p + "attn_q_norm.weight"));
            L.k_norm = f32(need(p + "attn_k_norm.weight"));
            L.swa = swa[il];
            L.ai = n_attn++;
            if (k) n_head_kv = (int)(k->ne[1] / head_dim);
        }
        const gtensor* fg = need(p + "ffn_gate.weight");
        const gtensor* fu = need(p + "ffn_up.weight");
        if (!fg || !fu) return false;
        n_ff = (int)fg->ne[1];
        std::vector<const uint8_t*> o;   // gate and up interleaved by 8-row group (seoul.cpp:155-160)
        for (int t = 0; t < n_ff; t += 8) { rows_of(o, fg, t, 8); rows_of(o, fu, t, 8); }
        ok &= (fg->type == T_Q4_0 || fg->type == T_Q4_1) && fu->type == fg->type &&
              q4_build(L.gate_up, o, (int)fg->ne[0], fg->type == T_Q4_1);
        ok &= whole(L.down, {need(p + "ffn_down.weight")});
        if (!ok) { fprintf(stderr, "oracle: layer %d has a table the kernels do not read\n", il); return false; }
    }
    if (!vocab_q6k && !whole(vocab, {tok})) return false;
    n_ctx = ctx_len;
    const int kvd = n_head_kv * head_dim;
    own.k_cache.assign(n_attn, std::vector<uint16_t>((size_t)n_ctx * kvd));
    own.v_cache.assign(n_attn, std::vector<uint16_t>((size_t)n_ctx * kvd));
    own.conv_state.assign(n_layer, {});
    for (int il = 0; il < n_layer; il++) if (layers[il].conv) own.conv_state[il].assign((size_t)n_embd * d_conv, 0.0f);
    own.hidden.assign(n_embd, 0.0f);
    own.logits.assign(n_vocab, 0.0f);
    n_threads = threads < 1 ? 1 : threads;
    per.resize(n_threads);
    const int wide = std::max({n_embd, n_ff, n_ctx});
    for (auto& T : per) { T.x.resize(n_embd); T.x2.resize(n_embd); T.h.resize(wide); T.t.resize(wide); T.u.resize(wide); }
    const int nqkv = n_head * head_dim + 2 * kvd + n_head;
    for (auto* v : {&bcx, &bcx2}) v->resize(3 * n_embd);
    for (auto* v : {&qkv, &qkv2}) v->resize(nqkv);
    for (auto* v : {&att, &att2}) v->resize(n_head * head_dim);
    for (auto* v : {&y, &y2, &fo, &fo2}) v->resize(n_embd);
    for (auto* v : {&act, &act2}) v->resize(n_ff);
    ctr.reset(new std::atomic<int>[n_ctr]);
    tm.start(n_threads);
    return true;
}

// input row: Q6_K word -> imi_q6k_dequant_row (seoul.cpp:363); Q4_0 word -> (code - 8) * d (ggml's
// dequantize_row_q4_0 semantics); or a given vector
void engine::embed(int32_t token, const float* embd, float* x) const {
    if (token >= 0 && vocab_q6k) {
        q6k_dequant_row(tok->data + (size_t)token * tok->row_bytes, x, n_embd / 256);
    } else if (token >= 0) {
        const uint8_t* row = tok->data + (size_t)token * tok->row_bytes;
        for (int j = 0; j < n_embd / 32; j++) {
            uint16_t dh; memcpy(&dh, row + 18 * j, 2);
            const float d = h2f(dh);
            const uint8_t* qs = row + 18 * j + 2;
            for (int i = 0; i < 16; i++) {
                x[32 * j + i] = (float)((qs[i] & 15) - 8) * d;
                x[32 * j + 16 + i] = (float)((qs[i] >> 4) - 8) * d;
            }
        }
    } else {
        memcpy(x, embd, (size_t)n_embd * sizeof(float));
    }
}

// word scores of one hidden state, rows taken from the shared counter k: Q6_K rows against the hidden state cut per
// 256 (seoul.cpp:479-487, chunks of 64 rows), or Q4_0 groups against it cut per 32
void engine::word_scores(per_thread& T, const float* hid, float* lg, std::atomic<int>& k) {
    if (vocab_q6k) {
        T.qk.from(hid, n_embd);
        const int nb = n_embd / 256, chunk = 64;
        for (int r = k.fetch_add(chunk, std::memory_order_relaxed); r < n_vocab; r = k.fetch_add(chunk, std::memory_order_relaxed))
            for (int i = r; i < std::min(n_vocab, r + chunk); i++) lg[i] = q6k_row(tok->data + (size_t)i * tok->row_bytes, T.qk, nb);
        return;
    }
    T.qi.from(hid, n_embd);
    const int ng = vocab.rows / 8;
    for (int g = k.fetch_add(4, std::memory_order_relaxed); g < ng; g = k.fetch_add(4, std::memory_order_relaxed))
        for (int gg = g; gg < std::min(ng, g + 4); gg++) q4_group(vocab, T.qi, gg, lg + 8 * gg);
}

state engine::new_state() const {   // imi/core/seoul.cpp:193-201
    state s;
    s.k_cache.assign(own.k_cache.size(), std::vector<uint16_t>(own.k_cache.empty() ? 0 : own.k_cache[0].size()));
    s.v_cache.assign(own.v_cache.size(), std::vector<uint16_t>(own.v_cache.empty() ? 0 : own.v_cache[0].size()));
    s.conv_state.assign(own.conv_state.size(), {});
    for (size_t i = 0; i < own.conv_state.size(); i++) s.conv_state[i].assign(own.conv_state[i].size(), 0.0f);
    s.hidden.assign(n_embd, 0.0f);
    s.logits.assign(n_vocab, 0.0f);
    return s;
}

// one (key/value head g, position p): k-norm, RoPE, fp16 cache write; then each of its query heads: q-norm, RoPE,
// scores, softmax (max subtracted, expf, double sum), weighted values, sigmoid head gate
// (imi/core/seoul.cpp:433-453, 291-315)
void engine::attend(const layer& L, const float* qv, uint16_t* kc, uint16_t* vc, int p, int g, float* at, float* sc) const {
    const int D = head_dim, kvd = n_head_kv * D, grp = n_head / n_head_kv, Hq = n_head * D;
    const float base = L.swa ? rope_base_swa : rope_base;
    const float* ff = L.swa ? nullptr : rope_freqs;
    const int s0 = (L.swa && n_swa > 0) ? std::max(0, p - n_swa + 1) : 0, nk = p - s0 + 1;
    const float scale = 1.0f / sqrtf((float)D);
    float kk[512];
    norm_mul(qv + Hq + g * D, L.k_norm, kk, D, eps);
    rope(kk, D, p, base, ff);
    const float* vv = qv + Hq + kvd + g * D;
    for (int i = 0; i < D; i++) { kc[(size_t)p * kvd + g * D + i] = f2h(kk[i]); vc[(size_t)p * kvd + g * D + i] = f2h(vv[i]); }
    for (int hh = 0; hh < grp; hh++) {
        const int h = g * grp + hh;
        float q[512], o[512];
        norm_mul(qv + h * D, L.q_norm, q, D, eps);
        rope(q, D, p, base, ff);
        float mx = -INFINITY;
        for (int t = 0; t < nk; t++) { sc[t] = dot_h(q, kc + (size_t)(s0 + t) * kvd + g * D, D) * scale; mx = std::max(mx, sc[t]); }
        double sum = 0;
        for (int t = 0; t < nk; t++) { sc[t] = expf(sc[t] - mx); sum += sc[t]; }
        const float inv = (float)(1.0 / sum);
        std::fill(o, o + D, 0.0f);
        for (int t = 0; t < nk; t++) axpy_h(sc[t] * inv, vc + (size_t)(s0 + t) * kvd + g * D, o, D);
        const float gate = 1.0f / (1.0f + expf(-qv[Hq + 2 * kvd + h]));
        for (int i = 0; i < D; i++) at[h * D + i] = o[i] * gate;
    }
}

void engine::step(int32_t token, const float* embd, bool want_logits) {   // imi/core/seoul.cpp:352-357
    if (own.pos >= n_ctx) { fprintf(stderr, "oracle: context full (%d)\n", n_ctx); return; }
    reset_counters();
    tm.run([&](int tid) { run(tid, token, embd, want_logits); });
    own.pos++;
}

// imi/core/seoul.cpp:359-488
void engine::run(int tid, int32_t token, const float* embd, bool want_logits) {
    per_thread& T = per[tid];
    const int E = n_embd, D = head_dim, Hq = n_head * D;
    float* x = T.x.data();
    embed(token, embd, x);
    int c = 0;
    auto table = [&](const q4tab& W, float* out) {
        std::atomic<int>& k = ctr[c++];
        const int ng = W.rows / 8;
        for (int g = k.fetch_add(4, std::memory_order_relaxed); g < ng; g = k.fetch_add(4, std::memory_order_relaxed))
            for (int gg = g; gg < std::min(ng, g + 4); gg++) q4_group(W, T.qi, gg, out + 8 * gg);
    };
    auto table_ffn = [&](const q4tab& W, float* out) {   // (gate, up) group pairs -> silu(gate) * up
        std::atomic<int>& k = ctr[c++];
        const int ng = W.rows / 8;
        float a[8], b[8];
        for (int g = k.fetch_add(4, std::memory_order_relaxed); g < ng; g = k.fetch_add(4, std::memory_order_relaxed))
            for (int gg = g; gg < std::min(ng, g + 4); gg += 2) {
                q4_group(W, T.qi, gg, a);
                q4_group(W, T.qi, gg + 1, b);
                float* o = out + 8 * (gg / 2);
                for (int i = 0; i < 8; i++) o[i] = silu(a[i]) * b[i];
            }
    };
    auto sync = [&] { tm.sync(); };
    auto cut = [&](const float* v, int n) {
        T.qi.from(v, n);
        if (tid == 0 && trace_cuts) cut_trace.insert(cut_trace.end(), T.qi.q.begin(), T.qi.q.begin() + n);
    };
    for (size_t il = 0; il < layers.size(); il++) {
        const layer& L = layers[il];
        norm_mul(x, L.attn_norm, T.h.data(), E, eps);
        cut(T.h.data(), E);
        if (L.conv) {
            table(L.in_proj, bcx.data());
            sync();
            const float *b = bcx.data(), *cc = b + E, *xx = b + 2 * E, *st = own.conv_state[il].data(), *w = L.conv_w.data();
            float* u = T.u.data();
            for (int e = 0; e < E; e++) u[e] = b[e] * xx[e] * w[d_conv * E + e];
            for (int k = 0; k < d_conv; k++) for (int e = 0; e < E; e++) u[e] = fmaf(st[k * E + e], w[k * E + e], u[e]);
            for (int e = 0; e < E; e++) u[e] *= cc[e];
            cut(u, E);
            table(L.out_proj, y.data());
            sync();
            if (tid == 0) {   // the conv memory slides one step
                float* sw = own.conv_state[il].data();
                memmove(sw, sw + E, (size_t)(d_conv - 1) * E * sizeof(float));
                for (int e = 0; e < E; e++) sw[(d_conv - 1) * E + e] = b[e] * xx[e];
            }
        } else {
            table(L.qkvg, qkv.data());
            sync();
            for (int g = tid; g < n_head_kv; g += n_threads)
                attend(L, qkv.data(), own.k_cache[L.ai].data(), own.v_cache[L.ai].data(), own.pos, g, att.data(), T.t.data());
            sync();
            cut(att.data(), Hq);
            table(L.o, y.data());
            sync();
        }
        norm_mul_add(y.data(), L.post_attn_norm, x, E, eps);
        norm_mul(x, L.ffn_norm, T.h.data(), E, eps);
        cut(T.h.data(), E);
        table_ffn(L.gate_up, act.data());
        sync();
        cut(act.data(), n_ff);
        table(L.down, fo.data());
        sync();
        norm_mul_add(fo.data(), L.post_ffn_norm, x, E, eps);
    }
    float* hid = T.h.data();
    norm_mul(x, out_norm, hid, E, eps);
    if (tid == 0) memcpy(own.hidden.data(), hid, (size_t)E * sizeof(float));
    if (want_logits) word_scores(T, hid, own.logits.data(), ctr[c++]);
    if (want_logits && !vocab_q6k && tid == 0 && trace_cuts)   // the word scores' cut of the hidden state
        cut_trace.insert(cut_trace.end(), T.qi.q.begin(), T.qi.q.begin() + E);
}

void engine::step2(int32_t ta, const float* ea, bool la, state& b, int32_t tb, const float* eb, bool lb) {   // seoul.cpp:208-220
    if (own.pos >= n_ctx || b.pos >= n_ctx) { fprintf(stderr, "oracle: context full (%d)\n", n_ctx); return; }
    reset_counters();
    const int32_t tk[2] = {ta, tb};
    const float* const em[2] = {ea, eb};
    const bool want[2] = {la, lb};
    tm.run([&](int tid) { run2(tid, b, tk, em, want); });
    own.pos++;
    b.pos++;
}

// imi/core/seoul.cpp:225-350: the same math per conversation; table reads shared through q4_group2
void engine::run2(int tid, state& B, const int32_t tk[2], const float* const em[2], const bool want[2]) {
    per_thread& T = per[tid];
    const int E = n_embd, Hq = n_head * head_dim;
    float* x[2] = {T.x.data(), T.x2.data()};
    q8in* qi[2] = {&T.qi, &T.qi2};
    float *bc[2] = {bcx.data(), bcx2.data()}, *qk[2] = {qkv.data(), qkv2.data()}, *at[2] = {att.data(), att2.data()};
    float *yy[2] = {y.data(), y2.data()}, *ac[2] = {act.data(), act2.data()}, *fq[2] = {fo.data(), fo2.data()};
    state* ss[2] = {&own, &B};
    for (int s = 0; s < 2; s++) embed(tk[s], em[s], x[s]);
    int c = 0;
    auto table2 = [&](const q4tab& W, float* o0, float* o1) {
        std::atomic<int>& k = ctr[c++];
        const int ng = W.rows / 8;
        for (int g = k.fetch_add(4, std::memory_order_relaxed); g < ng; g = k.fetch_add(4, std::memory_order_relaxed))
            for (int gg = g; gg < std::min(ng, g + 4); gg++) q4_group2(W, *qi[0], *qi[1], gg, o0 + 8 * gg, o1 + 8 * gg);
    };
    auto table_ffn2 = [&](const q4tab& W, float* o0, float* o1) {
        std::atomic<int>& k = ctr[c++];
        const int ng = W.rows / 8;
        float a0[8], a1[8], b0[8], b1[8];
        for (int g = k.fetch_add(4, std::memory_order_relaxed); g < ng; g = k.fetch_add(4, std::memory_order_relaxed))
            for (int gg = g; gg < std::min(ng, g + 4); gg += 2) {
                q4_group2(W, *qi[0], *qi[1], gg, a0, a1);
                q4_group2(W, *qi[0], *qi[1], gg + 1, b0, b1);
                float *p0 = o0 + 8 * (gg / 2), *p1 = o1 + 8 * (gg / 2);
                for (int i = 0; i < 8; i++) { p0[i] = silu(a0[i]) * b0[i]; p1[i] = silu(a1[i]) * b1[i]; }
            }
    };
    auto sync = [&] { tm.sync(); };
    for (size_t il = 0; il < layers.size(); il++) {
        const layer& L = layers[il];
        for (int s = 0; s < 2; s++) { norm_mul(x[s], L.attn_norm, T.h.data(), E, eps); qi[s]->from(T.h.data(), E); }
        if (L.conv) {
            table2(L.in_proj, bc[0], bc[1]);
            sync();
            for (int s = 0; s < 2; s++) {
                const float *b = bc[s], *cc = b + E, *xx = b + 2 * E, *st = ss[s]->conv_state[il].data(), *w = L.conv_w.data();
                float* u = T.u.data();
                for (int e = 0; e < E; e++) u[e] = b[e] * xx[e] * w[d_conv * E + e];
                for (int k = 0; k < d_conv; k++) for (int e = 0; e < E; e++) u[e] = fmaf(st[k * E + e], w[k * E + e], u[e]);
                for (int e = 0; e < E; e++) u[e] *= cc[e];
                qi[s]->from(u, E);
            }
            table2(L.out_proj, yy[0], yy[1]);
            sync();
            if (tid == 0)
                for (int s = 0; s < 2; s++) {
                    const float *b = bc[s], *xx = b + 2 * E;
                    float* sw = ss[s]->conv_state[il].data();
                    memmove(sw, sw + E, (size_t)(d_conv - 1) * E * sizeof(float));
                    for (int e = 0; e < E; e++) sw[(d_conv - 1) * E + e] = b[e] * xx[e];
                }
        } else {
            table2(L.qkvg, qk[0], qk[1]);
            sync();
            for (int u2 = tid; u2 < 2 * n_head_kv; u2 += n_threads) {   // (conversation, key/value head) pairs
                const int s = u2 / n_head_kv, g = u2 % n_head_kv;
                attend(L, qk[s], ss[s]->k_cache[L.ai].data(), ss[s]->v_cache[L.ai].data(), ss[s]->pos, g, at[s], T.t.data());
            }
            sync();
            for (int s = 0; s < 2; s++) qi[s]->from(at[s], Hq);
            table2(L.o, yy[0], yy[1]);
            sync();
        }
        for (int s = 0; s < 2; s++) {
            norm_mul_add(yy[s], L.post_attn_norm, x[s], E, eps);
            norm_mul(x[s], L.ffn_norm, T.h.data(), E, eps);
            qi[s]->from(T.h.data(), E);
        }
        table_ffn2(L.gate_up, ac[0], ac[1]);
        sync();
        for (int s = 0; s < 2; s++) qi[s]->from(ac[s], n_ff);
        table2(L.down, fq[0], fq[1]);
        sync();
        for (int s = 0; s < 2; s++) norm_mul_add(fq[s], L.post_ffn_norm, x[s], E, eps);
    }
    for (int s = 0; s < 2; s++) {
        float* hid = T.h.data();
        norm_mul(x[s], out_norm, hid, E, eps);
        if (tid == 0) memcpy(ss[s]->hidden.data(), hid, (size_t)E * sizeof(float));
        if (want[s]) word_scores(T, hid, ss[s]->logits.data(), ctr[c++]);
    }
}

// imi/core/seoul.cpp:490-517
void engine::step_batch(const int32_t* tokens, const float* embd, int n, bool want_logits, float* hidden_all) {
    if (bX.empty()) {
        const int kvd = n_head_kv * head_dim;
        bX.resize((size_t)NB * n_embd); bH.resize((size_t)NB * std::max(n_embd, n_ff)); bY.resize((size_t)NB * n_embd);
        bBig.resize((size_t)NB * std::max(3 * n_embd, n_head * head_dim + 2 * kvd + n_head)); bAct.resize((size_t)NB * n_ff);
    }
    for (int i0 = 0; i0 < n; i0 += NB) {
        const int m = std::min(NB, n - i0);
        if (own.pos + m > n_ctx) { fprintf(stderr, "oracle: context full (%d)\n", n_ctx); return; }
        reset_counters();
        tm.run([&](int tid) {
            run_batch(tid, tokens ? tokens + i0 : nullptr, embd ? embd + (size_t)i0 * n_embd : nullptr, m, hidden_all ? hidden_all + (size_t)i0 * n_embd : nullptr);
        });
        own.pos += m;
    }
    if (want_logits) {
        reset_counters();
        tm.run([&](int tid) { word_scores(per[tid], own.hidden.data(), own.logits.data(), ctr[0]); });
    }
}

// imi/core/seoul.cpp:519-655
void engine::run_batch(int tid, const int32_t* tokens, const float* embd, int n, float* hidden_all) {
    const int E = n_embd, D = head_dim, kvd = n_head_kv * D, grp = n_head / n_head_kv, nth = n_threads, Hq = n_head * D;
    const int p0 = tid * n / nth, p1 = (tid + 1) * n / nth;
    float *X = bX.data(), *H = bH.data(), *Y = bY.data(), *B = bBig.data(), *A = bAct.data();
    const int pos = own.pos;
    int c = 0;
    auto sync = [&] { tm.sync(); };
    auto table = [&](const q4tab& W, float* o, int ldo) {
        std::atomic<int>& k = ctr[c++];
        const int ng = W.rows / 8;
        float tmp[64 * 8];
        for (int g = k.fetch_add(1, std::memory_order_relaxed); g < ng; g = k.fetch_add(1, std::memory_order_relaxed)) {
            q4_group_batch(W, bq, g, tmp);
            for (int p = 0; p < n; p++) memcpy(o + (size_t)p * ldo + 8 * g, tmp + 8 * p, 8 * sizeof(float));
        }
    };
    auto table_ffn = [&](const q4tab& W, float* o) {
        std::atomic<int>& k = ctr[c++];
        const int ng = W.rows / 8;
        float a[64 * 8], b[64 * 8];
        for (int g = 2 * k.fetch_add(1, std::memory_order_relaxed); g < ng; g = 2 * k.fetch_add(1, std::memory_order_relaxed)) {
            q4_group_batch(W, bq, g, a);
            q4_group_batch(W, bq, g + 1, b);
            for (int p = 0; p < n; p++) { float* op = o + (size_t)p * n_ff + 4 * g; for (int r = 0; r < 8; r++) op[r] = silu(a[8 * p + r]) * b[8 * p + r]; }
        }
    };
    if (tid == 0) bq.shape(n, E);
    for (int p = p0; p < p1; p++) embed(tokens ? tokens[p] : -1, embd ? embd + (size_t)p * E : nullptr, X + (size_t)p * E);
    sync();
    for (size_t il = 0; il < layers.size(); il++) {
        const layer& L = layers[il];
        if (tid == 0) bq.shape(n, E);
        sync();
        for (int p = p0; p < p1; p++) { norm_mul(X + (size_t)p * E, L.attn_norm, H + (size_t)p * E, E, eps); bq.set(p, H + (size_t)p * E); }
        sync();
        if (L.conv) {
            table(L.in_proj, B, 3 * E);
            sync();
            const int e0 = tid * E / nth, e1 = (tid + 1) * E / nth;   // conv runs along positions, channels split
            float* st = own.conv_state[il].data();
            const float* w = L.conv_w.data();
            for (int p = 0; p < n; p++) {
                const float *b = B + (size_t)p * 3 * E, *cc = b + E, *xx = b + 2 * E;
                float* u = H + (size_t)p * E;
                for (int e = e0; e < e1; e++) {
                    const float bx = b[e] * xx[e];
                    float s = bx * w[(size_t)d_conv * E + e];
                    for (int k = 0; k < d_conv; k++) s = fmaf(st[(size_t)k * E + e], w[(size_t)k * E + e], s);
                    u[e] = cc[e] * s;
                    for (int k = 0; k + 1 < d_conv; k++) st[(size_t)k * E + e] = st[(size_t)(k + 1) * E + e];
                    st[(size_t)(d_conv - 1) * E + e] = bx;
                }
            }
            sync();
            for (int p = p0; p < p1; p++) bq.set(p, H + (size_t)p * E);
            sync();
            table(L.out_proj, Y, E);
            sync();
        } else {
            const int nr = Hq + 2 * kvd + n_head;
            table(L.qkvg, B, nr);
            sync();
            const float base = L.swa ? rope_base_swa : rope_base;
            const float* ff = L.swa ? nullptr : rope_freqs;
            uint16_t *kc = own.k_cache[L.ai].data(), *vc = own.v_cache[L.ai].data();
            for (int p = p0; p < p1; p++) {
                const float* r = B + (size_t)p * nr;
                for (int g = 0; g < n_head_kv; g++) {
                    float kk[512];
                    norm_mul(r + Hq + g * D, L.k_norm, kk, D, eps);
                    rope(kk, D, pos + p, base, ff);
                    for (int i = 0; i < D; i++) {
                        kc[(size_t)(pos + p) * kvd + g * D + i] = f2h(kk[i]);
                        vc[(size_t)(pos + p) * kvd + g * D + i] = f2h(r[Hq + kvd + g * D + i]);
                    }
                }
            }
            sync();
            const float scale = 1.0f / sqrtf((float)D);
            std::vector<float> sc(n_ctx);
            for (int u = tid; u < n * n_head; u += nth) {   // (position, head) pairs
                const int p = u / n_head, h = u % n_head, g = h / grp, at = pos + p;
                const int s0 = (L.swa && n_swa > 0) ? std::max(0, at - n_swa + 1) : 0, nk = at - s0 + 1;
                const float* r = B + (size_t)p * nr;
                float q[512], o[512];
                norm_mul(r + h * D, L.q_norm, q, D, eps);
                rope(q, D, at, base, ff);
                float mx = -INFINITY;
                for (int t = 0; t < nk; t++) { sc[t] = dot_h(q, kc + (size_t)(s0 + t) * kvd + g * D, D) * scale; mx = std::max(mx, sc[t]); }
                double sum = 0;
                for (int t = 0; t < nk; t++) { sc[t] = expf(sc[t] - mx); sum += sc[t]; }
                const float inv = (float)(1.0 / sum);
                std::fill(o, o + D, 0.0f);
                for (int t = 0; t < nk; t++) axpy_h(sc[t] * inv, vc + (size_t)(s0 + t) * kvd + g * D, o, D);
                const float gate = 1.0f / (1.0f + expf(-r[Hq + 2 * kvd + h]));
                float* out = H + (size_t)p * Hq + h * D;
                for (int i = 0; i < D; i++) out[i] = o[i] * gate;
            }
            sync();
            for (int p = p0; p < p1; p++) bq.set(p, H + (size_t)p * Hq);
            sync();
            table(L.o, Y, E);
            sync();
        }
        for (int p = p0; p < p1; p++) {
            norm_mul_add(Y + (size_t)p * E, L.post_attn_norm, X + (size_t)p * E, E, eps);
            norm_mul(X + (size_t)p * E, L.ffn_norm, H + (size_t)p * E, E, eps);
            bq.set(p, H + (size_t)p * E);
        }
        sync();
        table_ffn(L.gate_up, A);
        sync();
        if (tid == 0) bq.shape(n, n_ff);
        sync();
        for (int p = p0; p < p1; p++) bq.set(p, A + (size_t)p * n_ff);
        sync();
        table(L.down, Y, E);
        sync();
        for (int p = p0; p < p1; p++) norm_mul_add(Y + (size_t)p * E, L.post_ffn_norm, X + (size_t)p * E, E, eps);
        sync();
    }
    for (int p = p0; p < p1; p++) {
        float* hp = H + (size_t)p * E;
        norm_mul(X + (size_t)p * E, out_norm, hp, E, eps);
        if (hidden_all) memcpy(hidden_all + (size_t)p * E, hp, (size_t)E * sizeof(float));
        if (p == n - 1) memcpy(own.hidden.data(), hp, (size_t)E * sizeof(float));
    }
}

// ---------------------------------------------------------------- voice generator (imi/core/voice.{h,cpp})
struct voice {
    struct layer { const float *ln1, *ln2, *q_norm, *k_norm; q8gtab qkvg, o, gate_up, down; };
    gfile f;
    std::vector<layer> layers;
    q8gtab proj_in;
    std::vector<q8gtab> score;
    const gtensor *embd = nullptr, *out_embd = nullptr;
    const float *proj_b = nullptr, *mask_embd = nullptr, *out_norm = nullptr, *head_norm = nullptr;
    int n_embd = 0, n_vocab = 0, n_cb = 0, n_in = 0, n_head = 0, n_head_kv = 0, head_dim = 0, n_ff = 0, n_qkv = 0;
    float eps = 1e-5f, rope_theta = 1e6f;
    team tm;
    int n_threads = 1;
    std::vector<float> base, qkv, att, y, act;
    struct per_thread { std::vector<float> x, h, xt; };
    std::vector<per_thread> per;
    std::unique_ptr<std::atomic<int>[]> ctr;

    bool load(const std::string& path, int threads);
    void begin_frame(const float* h);
    void feedback(const int32_t* codes, float* out) const;
    void pass(const int32_t* codes, const std::vector<int>& need, float* out);
    void run_pass(int tid, const int32_t* codes, const std::vector<int>& need, float* out);
};

bool voice::load(const std::string& path, int threads) {   // imi/core/voice.cpp:78-139
    if (!f.open(path)) return false;
    const std::string g = "a.gen.code.";
    embd = f.get(g + "embd.weight");
    out_embd = f.get(g + "out_embd.weight");
    mask_embd = f32(f.get(g + "mask_embd"));
    out_norm = f32(f.get(g + "output_norm.weight"));
    head_norm = f32(f.get(g + "head_norm.weight"));
    proj_b = f32(f.get(g + "proj_in.bias"));
    const gtensor* pw = f.get(g + "proj_in.weight");
    if (!embd || !out_embd || !mask_embd || !out_norm || !head_norm || !proj_b || !pw) { fprintf(stderr, "oracle: generator tensor missing\n"); return false; }
    if (embd->type != T_Q8_0) { fprintf(stderr, "oracle: generator needs 8-bit tables\n"); return false; }
    n_embd = (int)embd->ne[0]; n_vocab = (int)embd->ne[1]; n_cb = (int)embd->ne[2]; n_in = (int)pw->ne[0];
    auto rows_of = [](std::vector<const uint8_t*>& o, const gtensor* t, int r0, int n, int plane) {
        for (int r = r0; r < r0 + n; r++) o.push_back(t->data + (size_t)plane * t->row_bytes * t->ne[1] + (size_t)r * t->row_bytes);
    };
    auto whole = [&](q8gtab& dst, std::vector<const gtensor*> parts) {
        std::vector<const uint8_t*> o;
        for (auto* p : parts) { if (!p || p->type != T_Q8_0) return false; rows_of(o, p, 0, (int)p->ne[1], 0); }
        return q8g_build(dst, o, (int)parts[0]->ne[0]);
    };
    bool ok = whole(proj_in, {pw});
    for (int il = 0;; il++) {
        const std::string p = g + "blk." + std::to_string(il) + ".";
        if (!f.get(p + "ln1.weight")) break;
        layer L;
        L.ln1 = f32(f.get(p + "ln1.weight")); L.ln2 = f32(f.get(p + "ln2.weight"));
        L.q_norm = f32(f.get(p + "attn_q_norm.weight")); L.k_norm = f32(f.get(p + "attn_k_norm.weight"));
        const gtensor *q = f.get(p + "attn_q.weight"), *k = f.get(p + "attn_k.weight");
        if (!q || !k || !L.q_norm) return false;
        head_dim = (int)f.get(p + "attn_q_norm.weight")->ne[0];
        n_head = (int)(q->ne[1] / head_dim); n_head_kv = (int)(k->ne[1] / head_dim);
        ok &= whole(L.qkvg, {q, k, f.get(p + "attn_v.weight"), f.get(p + "attn_gate.weight")});
        ok &= whole(L.o, {f.get(p + "attn_out.weight")});
        const gtensor *fg = f.get(p + "ffn_gate.weight"), *fu = f.get(p + "ffn_up.weight");
        if (!fg || !fu) return false;
        n_ff = (int)fg->ne[1];
        std::vector<const uint8_t*> o;
        for (int t = 0; t < n_ff; t += 8) { rows_of(o, fg, t, 8, 0); rows_of(o, fu, t, 8, 0); }
        ok &= q8g_build(L.gate_up, o, (int)fg->ne[0]);
        ok &= whole(L.down, {f.get(p + "ffn_down.weight")});
        layers.push_back(std::move(L));
    }
    score.resize(n_cb);
    for (int c = 0; c < n_cb; c++) {
        std::vector<const uint8_t*> o;
        rows_of(o, embd, 0, n_vocab, c);
        ok &= q8g_build(score[c], o, n_embd);
    }
    if (!ok) { fprintf(stderr, "oracle: a generator table is not 8-bit\n"); return false; }
    n_qkv = (n_head + 2 * n_head_kv) * head_dim + n_head;
    n_threads = threads < 1 ? 1 : threads;
    per.resize(n_threads);
    const int wide = std::max({n_embd, n_ff, n_in});
    for (auto& T : per) { T.x.resize((size_t)n_cb * n_embd); T.h.resize((size_t)n_cb * wide); T.xt.resize((size_t)n_cb * wide); }
    qkv.resize((size_t)n_cb * n_qkv); att.resize((size_t)n_cb * n_head * head_dim); y.resize((size_t)n_cb * n_embd);
    act.resize((size_t)n_cb * n_ff); base.resize((size_t)n_cb * n_embd);
    ctr.reset(new std::atomic<int>[64]);
    tm.start(n_threads);
    return true;
}
void voice::feedback(const int32_t* codes, float* out) const {   // voice.cpp:141-148
    std::vector<float> row(n_in);
    std::fill(out, out + n_in, 0.0f);
    for (int c = 0; c < n_cb; c++) {
        q8_0_dequant_row(out_embd->data + (size_t)(codes[c] + c * n_vocab) * out_embd->row_bytes, row.data(), n_in);
        for (int i = 0; i < n_in; i++) out[i] += row[i];
    }
}
void voice::begin_frame(const float* h) {   // voice.cpp:150-162
    ctr[0].store(0);
    tm.run([&](int) {
        const int ng = proj_in.rows_pad / 8;
        float o[8];
        for (int g = ctr[0].fetch_add(8); g < ng; g = ctr[0].fetch_add(8))
            for (int gg = g; gg < std::min(ng, g + 8); gg++) {
                q8g_group(proj_in, h, 1, gg, o);
                for (int r = 0; r < 8; r++) base[8 * gg + r] = o[r] + proj_b[8 * gg + r];
            }
    });
}
void voice::pass(const int32_t* codes, const std::vector<int>& need, float* out) {   // voice.cpp:164-168
    for (int i = 0; i < 64; i++) ctr[i].store(0, std::memory_order_relaxed);
    tm.run([&](int tid) { run_pass(tid, codes, need, out); });
}
static void transpose(const float* a, int P, int K, int lda, float* t) {
    for (int p = 0; p < P; p++) for (int k = 0; k < K; k++) t[(size_t)k * P + p] = a[(size_t)p * lda + k];
}
// imi/core/voice.cpp:170-257
void voice::run_pass(int tid, const int32_t* codes, const std::vector<int>& need, float* out) {
    per_thread& T = per[tid];
    const int E = n_embd, P = n_cb, D = head_dim, Hq = n_head * D, Hk = n_head_kv * D, grp = n_head / n_head_kv;
    float *x = T.x.data(), *h = T.h.data(), *xt = T.xt.data();
    for (int i = 0; i < P; i++) {
        float* row = x + (size_t)i * E;
        if (codes[i] >= 0) q8_0_dequant_row(embd->data + (size_t)i * embd->row_bytes * embd->ne[1] + (size_t)codes[i] * embd->row_bytes, row, E);
        else memcpy(row, mask_embd, (size_t)E * sizeof(float));
        for (int e = 0; e < E; e++) row[e] += base[(size_t)i * E + e];
    }
    int c = 0;
    auto table = [&](const q8gtab& W, float* o, int ldo) {
        std::atomic<int>& k = ctr[c++];
        const int ng = W.rows_pad / 8;
        float tmp[64 * 8];
        for (int g = k.fetch_add(2, std::memory_order_relaxed); g < ng; g = k.fetch_add(2, std::memory_order_relaxed))
            for (int gg = g; gg < std::min(ng, g + 2); gg++) {
                q8g_group(W, xt, P, gg, tmp);
                for (int p = 0; p < P; p++) for (int r = 0; r < 8 && 8 * gg + r < W.rows; r++) o[(size_t)p * ldo + 8 * gg + r] = tmp[8 * p + r];
            }
    };
    auto table_ffn = [&](const q8gtab& W, float* o) {
        std::atomic<int>& k = ctr[c++];
        const int ng = W.rows_pad / 8;
        float a[64 * 8], b[64 * 8];
        for (int g = k.fetch_add(2, std::memory_order_relaxed); g < ng; g = k.fetch_add(2, std::memory_order_relaxed)) {
            q8g_group(W, xt, P, g, a);
            q8g_group(W, xt, P, g + 1, b);
            for (int p = 0; p < P; p++) for (int r = 0; r < 8; r++) o[(size_t)p * n_ff + 4 * g + r] = silu(a[8 * p + r]) * b[8 * p + r];
        }
    };
    for (const layer& L : layers) {
        for (int p = 0; p < P; p++) norm_mul(x + (size_t)p * E, L.ln1, h + (size_t)p * E, E, eps);
        transpose(h, P, E, E, xt);
        table(L.qkvg, qkv.data(), n_qkv);
        tm.sync();
        for (int hh = tid; hh < n_head; hh += n_threads) {   // each thread: whole query heads
            const int kv = hh / grp;
            float kk[64][64], qq[64][64], sc[64];
            for (int p = 0; p < P; p++) {
                const float* r = qkv.data() + (size_t)p * n_qkv;
                norm_mul(r + Hq + kv * D, L.k_norm, kk[p], D, eps); rope(kk[p], D, p, rope_theta, nullptr);
                norm_mul(r + hh * D, L.q_norm, qq[p], D, eps); rope(qq[p], D, p, rope_theta, nullptr);
            }
            const float scale = 1.0f / sqrtf((float)D);
            for (int p = 0; p < P; p++) {
                float mx = -INFINITY;
                for (int t = 0; t < P; t++) {
                    float s = 0.0f;
                    for (int i = 0; i < D; i++) s = fmaf(qq[p][i], kk[t][i], s);
                    sc[t] = s * scale;
                    mx = std::max(mx, sc[t]);
                }
                float sum = 0.0f;
                for (int t = 0; t < P; t++) { sc[t] = expf(sc[t] - mx); sum += sc[t]; }
                const float gate = 1.0f / (1.0f + expf(-qkv[(size_t)p * n_qkv + Hq + 2 * Hk + hh]));
                float* o = att.data() + (size_t)p * Hq + hh * D;
                for (int i = 0; i < D; i++) {
                    float a = 0.0f;
                    for (int t = 0; t < P; t++) a = fmaf(sc[t], qkv[(size_t)t * n_qkv + Hq + Hk + kv * D + i], a);
                    o[i] = a / sum * gate;
                }
            }
        }
        tm.sync();
        transpose(att.data(), P, Hq, Hq, xt);
        table(L.o, y.data(), E);
        tm.sync();
        for (size_t i = 0; i < (size_t)P * E; i++) x[i] += y[i];
        for (int p = 0; p < P; p++) norm_mul(x + (size_t)p * E, L.ln2, h + (size_t)p * E, E, eps);
        transpose(h, P, E, E, xt);
        table_ffn(L.gate_up, act.data());
        tm.sync();
        transpose(act.data(), P, n_ff, n_ff, xt);
        table(L.down, y.data(), E);
        tm.sync();
        for (size_t i = 0; i < (size_t)P * E; i++) x[i] += y[i];
    }
    for (int p = 0; p < P; p++) {
        norm_mul(x + (size_t)p * E, out_norm, h + (size_t)p * E, E, eps);
        norm_mul(h + (size_t)p * E, head_norm + (size_t)p * E, xt + (size_t)p * E, E, eps);
    }
    std::atomic<int>& k = ctr[c++];
    const int ng = score[0].rows_pad / 8, units = (int)need.size() * ng;
    float tmp[8];
    for (int u = k.fetch_add(4, std::memory_order_relaxed); u < units; u = k.fetch_add(4, std::memory_order_relaxed))
        for (int uu = u; uu < std::min(units, u + 4); uu++) {
            const int j = uu / ng, gg = uu % ng, cb = need[j];
            q8g_group(score[cb], xt + (size_t)cb * E, 1, gg, tmp);
            for (int r = 0; r < 8 && 8 * gg + r < n_vocab; r++) out[(size_t)j * n_vocab + 8 * gg + r] = tmp[r];
        }
}

}  // namespace orc

// ---------------------------------------------------------------- C API for the tests (ctypes)
using namespace orc;
extern "C" {

void* orc_engine_load(const char* path, int threads, int n_ctx) {
    auto* e = new engine;
    if (!e->load(path, threads, n_ctx)) { delete e; return nullptr; }
    return e;
}
void orc_engine_free(void* h) { delete (engine*)h; }
// n_embd, n_vocab, n_head, n_head_kv, head_dim, n_ff, d_conv, n_ctx, n_layer, n_swa, pos, n_threads
void orc_engine_info(void* h, int* o) {
    auto* e = (engine*)h;
    const int v[12] = {e->n_embd, e->n_vocab, e->n_head, e->n_head_kv, e->head_dim, e->n_ff, e->d_conv, e->n_ctx, (int)e->layers.size(), e->n_swa, e->own.pos, e->n_threads};
    memcpy(o, v, sizeof(v));
}
void orc_engine_reset(void* h) {   // imi/core/seoul.cpp:188-191
    auto* e = (engine*)h;
    e->own.pos = 0;
    for (auto& s : e->own.conv_state) std::fill(s.begin(), s.end(), 0.0f);
}
void orc_engine_set_pos(void* h, int pos) { ((engine*)h)->own.pos = pos; }
void orc_engine_step(void* h, int token, const float* embd, int want_logits, float* hidden, float* logits) {
    auto* e = (engine*)h;
    e->step(token, embd, want_logits != 0);
    if (hidden) memcpy(hidden, e->own.hidden.data(), e->n_embd * sizeof(float));
    if (logits && want_logits) memcpy(logits, e->own.logits.data(), (size_t)e->n_vocab * sizeof(float));
}
void* orc_state_new(void* h) { return new state(((engine*)h)->new_state()); }
void orc_state_free(void* s) { delete (state*)s; }
void orc_state_info(void* s, int* pos) { *pos = ((state*)s)->pos; }
void orc_swap_state(void* h, void* s) {   // imi/core/seoul.cpp:203-206
    auto* e = (engine*)h; auto* b = (state*)s;
    e->own.k_cache.swap(b->k_cache); e->own.v_cache.swap(b->v_cache); e->own.conv_state.swap(b->conv_state);
    std::swap(e->own.pos, b->pos); e->own.hidden.swap(b->hidden); e->own.logits.swap(b->logits);
}
void orc_engine_step2(void* h, int ta, const float* ea, int la, void* sb, int tb, const float* eb, int lb,
                      float* hid_a, float* lg_a, float* hid_b, float* lg_b) {
    auto* e = (engine*)h; auto* b = (state*)sb;
    e->step2(ta, ea, la != 0, *b, tb, eb, lb != 0);
    if (hid_a) memcpy(hid_a, e->own.hidden.data(), e->n_embd * sizeof(float));
    if (lg_a && la) memcpy(lg_a, e->own.logits.data(), (size_t)e->n_vocab * sizeof(float));
    if (hid_b) memcpy(hid_b, b->hidden.data(), e->n_embd * sizeof(float));
    if (lg_b && lb) memcpy(lg_b, b->logits.data(), (size_t)e->n_vocab * sizeof(float));
}
void orc_engine_step_batch(void* h, const int* tokens, const float* embd, int n, int want_logits, float* hidden_last, float* logits, float* hidden_all) {
    auto* e = (engine*)h;
    e->step_batch(tokens, embd, n, want_logits != 0, hidden_all);
    if (hidden_last) memcpy(hidden_last, e->own.hidden.data(), e->n_embd * sizeof(float));
    if (logits && want_logits) memcpy(logits, e->own.logits.data(), (size_t)e->n_vocab * sizeof(float));
}
static int argmax_first(const float* a, int n) { int t = 0; for (int i = 1; i < n; i++) if (a[i] > a[t]) t = i; return t; }
// greedy decode timing: n_steps steps from the current state, feeding back the argmax; returns seconds
double orc_engine_greedy(void* h, int first_token, int n_steps, int* out_tokens) {
    auto* e = (engine*)h;
    int tok = first_token;
    const auto t0 = std::chrono::steady_clock::now();
    for (int i = 0; i < n_steps; i++) {
        e->step(tok, nullptr, true);
        tok = argmax_first(e->own.logits.data(), e->n_vocab);
        if (out_tokens) out_tokens[i] = tok;
    }
    return std::chrono::duration<double>(std::chrono::steady_clock::now() - t0).count();
}
double orc_engine_greedy2(void* h, void* sb, int ta, int tb, int n_steps, int* out_a, int* out_b) {
    auto* e = (engine*)h; auto* b = (state*)sb;
    const auto t0 = std::chrono::steady_clock::now();
    for (int i = 0; i < n_steps; i++) {
        e->step2(ta, nullptr, true, *b, tb, nullptr, true);
        ta = argmax_first(e->own.logits.data(), e->n_vocab);
        tb = argmax_first(b->logits.data(), e->n_vocab);
        if (out_a) out_a[i] = ta;
        if (out_b) out_b[i] = tb;
    }
    return std::chrono::duration<double>(std::chrono::steady_clock::now() - t0).count();
}
// K/V cache and conv state of the engine's own conversation, for state checks
void orc_engine_cache(void* h, int ai, uint16_t* k, uint16_t* v) {
    auto* e = (engine*)h;
    memcpy(k, e->own.k_cache[ai].data(), e->own.k_cache[ai].size() * 2);
    memcpy(v, e->own.v_cache[ai].data(), e->own.v_cache[ai].size() * 2);
}
// the cut trace of single steps: on != 0 starts it (empty), on == 0 stops it; take copies out up to cap codes, clears
// the trace and returns how many it held (out == nullptr: only the count, nothing cleared)
void orc_engine_trace_cuts(void* h, int on) {
    auto* e = (engine*)h;
    e->trace_cuts = on != 0;
    e->cut_trace.clear();
}
size_t orc_engine_take_cuts(void* h, int8_t* out, size_t cap) {
    auto* e = (engine*)h;
    const size_t n = e->cut_trace.size();
    if (!out) return n;
    memcpy(out, e->cut_trace.data(), std::min(n, cap));
    e->cut_trace.clear();
    return n;
}
void orc_engine_conv_state(void* h, int il, float* out) {
    auto* e = (engine*)h;
    memcpy(out, e->own.conv_state[il].data(), e->own.conv_state[il].size() * sizeof(float));
}

// ---- kernel-level entry points ----
float orc_h2f(uint16_t h) { return h2f(h); }
// Q6_K word table pieces: x [n] -> codes, d [n/256], bsums [n/16]; rows of nblocks 210-byte blocks
void orc_q8k_from(const float* x, int n, int8_t* q, float* d, int16_t* bsums) {
    q8kin X;
    X.from(x, n);
    memcpy(q, X.q.data(), (size_t)n);
    memcpy(d, X.d.data(), sizeof(float) * (size_t)(n / 256));
    memcpy(bsums, X.bsums.data(), sizeof(int16_t) * (size_t)(n / 16));
}
void orc_q6k_dequant_row(const uint8_t* row, int nblocks, float* y) { q6k_dequant_row(row, y, nblocks); }
void orc_q6k_rows(const uint8_t* rows, int n_rows, int nblocks, const float* x, float* out, int32_t* lanes) {
    q8kin X;
    X.from(x, 256 * nblocks);
    for (int r = 0; r < n_rows; r++) {
        const uint8_t* row = rows + (size_t)r * 210 * nblocks;
        out[r] = q6k_row(row, X, nblocks);
        if (lanes)
            for (int i = 0; i < nblocks; i++) q6k_lane_sums(row + 210 * (size_t)i, X, i, lanes + ((size_t)r * nblocks + i) * 8);
    }
}
uint16_t orc_f2h(float f) { return f2h(f); }
float orc_cut32(const float* x, int8_t* q, int* sum) { return cut32(x, q, sum); }
void orc_cut(const float* x, int n, int8_t* q, float* d, float* s) {
    q8in X; X.from(x, n);
    memcpy(q, X.q.data(), n); memcpy(d, X.d.data(), n / 32 * 4); memcpy(s, X.s.data(), n / 32 * 4);
}
// imi 8-row layout of a Q4_0 matrix [rows][cols] (rows % 8 == 0)
void orc_q4_layout(const uint8_t* q4_0, int rows, int cols, uint8_t* codes, uint16_t* d) {
    std::vector<const uint8_t*> rr(rows);
    for (int r = 0; r < rows; r++) rr[r] = q4_0 + (size_t)r * (cols / 32) * 18;
    q4tab t; q4_build(t, rr, cols);
    memcpy(codes, t.codes.data(), t.codes.size()); memcpy(d, t.d.data(), t.d.size() * 2);
}
struct q4h { q4tab t; team tm; };
// q4_1: the rows are Q4_1 (20-byte blocks)
void* orc_q4_create(const uint8_t* q4, int rows, int cols, int threads, int q4_1) {
    auto* h = new q4h;
    std::vector<const uint8_t*> rr(rows);
    for (int r = 0; r < rows; r++) rr[r] = q4 + (size_t)r * (cols / 32) * (q4_1 ? 20 : 18);
    if (!q4_build(h->t, rr, cols, q4_1 != 0)) { delete h; return nullptr; }
    h->tm.start(threads);
    return h;
}
void orc_q4_free(void* h) { delete (q4h*)h; }
// y[n_in][rows] = W x_i for n_in in {1, 2} (group / group2), cut per thread as imi does; mode 1 = scalar restatement.
// Returns the best wall time in seconds over reps.
double orc_q4_gemv(void* hh, const float* x, int n_in, float* y, int mode, int reps) {
    auto* h = (q4h*)hh;
    const q4tab& W = h->t;
    const int ng = W.rows / 8;
    double best = 1e30;
    for (int rep = 0; rep < std::max(1, reps); rep++) {
        std::atomic<int> next{0};
        const auto t0 = std::chrono::steady_clock::now();
        h->tm.run([&](int) {
            q8in X, X2;
            X.from(x, W.cols);
            if (n_in > 1) X2.from(x + W.cols, W.cols);
            for (int g = next.fetch_add(4); g < ng; g = next.fetch_add(4))
                for (int gg = g; gg < std::min(ng, g + 4); gg++) {
                    if (mode == 1) { q4_group_scalar(W, X, gg, y + 8 * gg); if (n_in > 1) q4_group_scalar(W, X2, gg, y + W.rows + 8 * gg); }
                    else if (n_in > 1) q4_group2(W, X, X2, gg, y + 8 * gg, y + W.rows + 8 * gg);
                    else q4_group(W, X, gg, y + 8 * gg);
                }
        });
        best = std::min(best, std::chrono::duration<double>(std::chrono::steady_clock::now() - t0).count());
    }
    return best;
}
// n inputs (n <= 64) through the batch kernel: x [n][cols] -> y [n][rows]
void orc_q4_gemv_batch(void* hh, const float* x, int n, float* y) {
    auto* h = (q4h*)hh;
    const q4tab& W = h->t;
    q8b X; X.shape(n, W.cols);
    for (int i = 0; i < n; i++) X.set(i, x + (size_t)i * W.cols);
    std::vector<float> tmp(64 * 8);
    for (int g = 0; g < W.rows / 8; g++) {
        q4_group_batch(W, X, g, tmp.data());
        for (int i = 0; i < n; i++) memcpy(y + (size_t)i * W.rows + 8 * g, tmp.data() + 8 * i, 32);
    }
}
void orc_q4_block_sums(void* hh, const float* x, int32_t* sums) {   // [rows][nb] integer block sums
    auto* h = (q4h*)hh;
    q8in X; X.from(x, h->t.cols);
    for (int g = 0; g < h->t.rows / 8; g++) q4_block_sums(h->t, X, g, sums + (size_t)g * 8 * h->t.nb);
}
struct q4x8h { q4x8tab t; team tm; };
void* orc_q4x8_create(const uint8_t* q4_0, int rows, int cols, int threads) {
    auto* h = new q4x8h;
    q4x8_build(h->t, q4_0, rows, cols);
    h->tm.start(threads);
    return h;
}
void orc_q4x8_free(void* h) { delete (q4x8h*)h; }
// imi/kernels/q4x8.cpp:80-94: every thread cuts the input, then 32-row chunks from a shared counter
double orc_q4x8_gemv(void* hh, const float* x, float* y, int reps) {
    auto* h = (q4x8h*)hh;
    const int ng = h->t.rows / 8;
    double best = 1e30;
    for (int rep = 0; rep < std::max(1, reps); rep++) {
        std::atomic<int> next{0};
        const auto t0 = std::chrono::steady_clock::now();
        h->tm.run([&](int) {
            q4x8in X;
            q4x8_quant_in(x, h->t.cols, X);
            for (int g = next.fetch_add(4); g < ng; g = next.fetch_add(4)) q4x8_rows(h->t, X, y, g, std::min(ng, g + 4));
        });
        best = std::min(best, std::chrono::duration<double>(std::chrono::steady_clock::now() - t0).count());
    }
    return best;
}
void orc_q4x8_layout(void* hh, uint8_t* codes, float* scales) {
    auto* h = (q4x8h*)hh;
    memcpy(codes, h->t.codes.data(), h->t.codes.size()); memcpy(scales, h->t.scales.data(), h->t.scales.size() * 4);
}
void orc_q4x8_quant_in(const float* x, int n, int8_t* q, float* d, float* corr) {
    q4x8in X; q4x8_quant_in(x, n, X);
    memcpy(q, X.q.data(), n); memcpy(d, X.d.data(), n / 32 * 4); memcpy(corr, X.corr.data(), n / 32 * 4);
}
// Q8_0 k-major group kernel: W Q8_0 [rows][cols], xt [cols][C] -> out [C][rows_pad]
void orc_q8g_gemm(const uint8_t* q8_0, int rows, int cols, const float* xt, int C, float* out) {
    std::vector<const uint8_t*> rr(rows);
    for (int r = 0; r < rows; r++) rr[r] = q8_0 + (size_t)r * (cols / 32) * 34;
    q8gtab t; q8g_build(t, rr, cols);
    std::vector<float> tmp((size_t)C * 8);
    for (int g = 0; g < t.rows_pad / 8; g++) {
        q8g_group(t, xt, C, g, tmp.data());
        for (int c = 0; c < C; c++) memcpy(out + (size_t)c * t.rows_pad + 8 * g, tmp.data() + 8 * c, 32);
    }
}
float orc_rms_scale(const float* x, int n, float eps) { return rms_scale(x, n, eps); }
void orc_expf(const float* x, long long n, float* y) { for (long long i = 0; i < n; i++) y[i] = expf(x[i]); }   // the C library's
void orc_rope(float* v, int n, int pos, float base, const float* ff) { rope(v, n, pos, base, ff); }

// ---- voice generator ----
void* orc_voice_load(const char* path, int threads) {
    auto* v = new voice;
    if (!v->load(path, threads)) { delete v; return nullptr; }
    return v;
}
void orc_voice_free(void* h) { delete (voice*)h; }
void orc_voice_info(void* h, int* o) {   // n_embd, n_vocab, n_cb, n_in, n_head, n_head_kv, head_dim, n_ff, n_layer
    auto* v = (voice*)h;
    const int a[9] = {v->n_embd, v->n_vocab, v->n_cb, v->n_in, v->n_head, v->n_head_kv, v->head_dim, v->n_ff, (int)v->layers.size()};
    memcpy(o, a, sizeof(a));
}
void orc_voice_begin_frame(void* h, const float* hid) { ((voice*)h)->begin_frame(hid); }
void orc_voice_base(void* h, float* out) { auto* v = (voice*)h; memcpy(out, v->base.data(), v->base.size() * 4); }
void orc_voice_pass(void* h, const int32_t* codes, const int32_t* need, int n_need, float* out) {
    std::vector<int> nd(need, need + n_need);
    ((voice*)h)->pass(codes, nd, out);
}
void orc_voice_feedback(void* h, const int32_t* codes, float* out) { ((voice*)h)->feedback(codes, out); }

// imi_talker::next's pick of one codebook (imi/core/talk.cpp:147-164) for each score row j of a pass: the repeat
// penalty over the history window (each distinct code once), then temperature probabilities in double, their sum
// in code order, keep = 1 - p[eos] / sum, and the pick by subtracting p in code order from r = u * sum. The
// uniform draw u[j] replaces imi's std::uniform_real_distribution<double>(0, 1)(rng); rows are penalised in place.
void orc_voice_sample(float* scores, int n, int V, const int32_t* cbs, const int32_t* hist, int n_frames, int n_cb,
                      const double* u, float temp, float rep, int32_t* picks, double* keep) {
    const int eos = V - 1;
    std::vector<char> seen(V);
    std::vector<double> p(V);
    for (int j = 0; j < n; j++) {
        float* l = scores + (size_t)j * V;
        const int cb = cbs[j];
        std::fill(seen.begin(), seen.end(), 0);
        for (int f = 0; f < n_frames; f++) {
            const int c = hist[(size_t)f * n_cb + cb];
            if (c >= 0 && c < V && !seen[c]) { seen[c] = 1; l[c] = l[c] > 0 ? l[c] / rep : l[c] * rep; }
        }
        const float lmax = *std::max_element(l, l + V);
        double sum = 0;
        for (int v = 0; v < V; v++) { p[v] = std::exp((double)(l[v] - lmax) / temp); sum += p[v]; }
        keep[j] = 1.0 - p[eos] / sum;
        double r = u[j] * sum;
        int pick = V - 1;
        for (int v = 0; v < V; v++) { r -= p[v]; if (r <= 0) { pick = v; break; } }
        picks[j] = pick;
    }
}

}  // extern "C"
