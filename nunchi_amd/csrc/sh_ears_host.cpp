// Host side of the ears on the device (imi/core/ears.{h,cpp}): load (the float tables in the device layout, the mel
// front end's Hann window, DFT table and Slaney filters built as imi builds them), the encode launch sequence, and
// the C ABI.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstring>
#include <string>
#include <vector>

#include "../../include/seoul_hip.h"
#include "gguf_file.h"
#include "sh_ears.h"

namespace sh {
int set_error(int code, const std::string& msg);
}
using namespace sh;

namespace {
#define ECHK(x)                                                                                                 \
    do {                                                                                                        \
        hipError_t e_ = (x);                                                                                    \
        if (e_ != hipSuccess) return set_error(SH_E_HIP, std::string(#x) + ": " + hipGetErrorString(e_));       \
    } while (0)

struct elayer {
    bool attn = false;
    const float *ln1 = nullptr, *ln2 = nullptr, *conv_w = nullptr, *q_norm = nullptr, *k_norm = nullptr;
    etab in, out, gate_up, down;
};

constexpr int N_FFT = 400, HOP = 160, N_BIN = N_FFT / 2 + 1;

inline int pad16(long v) { return (int)((v + 15) / 16 * 16); }

struct geom {   // imi/core/ears.cpp:201-205
    int n_fr, T2, F2, T4, F4, P, F8;
};
geom geometry(int n, int n_mel) {
    const int n_pad = n <= N_FFT ? N_FFT : n + (HOP - (n - N_FFT) % HOP) % HOP;
    geom g{};
    g.n_fr = (n_pad - N_FFT) / HOP + 1;
    g.T2 = (g.n_fr + 1) / 2; g.F2 = n_mel / 2;
    g.T4 = (g.T2 + 1) / 2; g.F4 = g.F2 / 2;
    g.P = (g.T4 + 1) / 2; g.F8 = g.F4 / 2;
    return g;
}
}  // namespace

struct sh_ears {
    int device = 0;
    hipStream_t stream = nullptr;
    sh_ears_shape info{};
    float eps = 1e-5f, theta = 1e6f;
    char* mem = nullptr;   // weights
    std::vector<elayer> layers;
    etab dft, c3, c6, pre, mlp1, mlp3;
    const int2* fb_span = nullptr;   // per mel: the filter's nonzero bins [lo, hi)
    const float *hann = nullptr, *fb = nullptr, *c0_w = nullptr, *c0_b = nullptr, *c2_w = nullptr, *c2_b = nullptr,
                *c3_b = nullptr, *c5_w = nullptr, *c5_b = nullptr, *c6_b = nullptr, *pre_b = nullptr,
                *post_ln = nullptr, *ln_w = nullptr, *ln_b = nullptr, *mlp1_b = nullptr, *mlp3_b = nullptr;
    int n_mid = 0;         // projector width (mlp.1 rows)
    int big_w = 0;         // widest layer input table (3 n_embd or q|k|v)
    // work, grown on demand
    char* work = nullptr;
    size_t work_cap = 0;
    float *pcm = nullptr, *fx = nullptr, *pw = nullptr, *mel = nullptr, *a0 = nullptr, *a1 = nullptr, *a2 = nullptr,
          *a3 = nullptr, *a4 = nullptr, *xf = nullptr, *x = nullptr, *h = nullptr, *big = nullptr, *act = nullptr,
          *proj = nullptr, *out = nullptr;
    float2* cs = nullptr;
    float* host_in = nullptr;   // pinned staging: samples in, rows out, rope table
    size_t host_cap = 0;
    int last_frames = 0;
};

namespace {

void release(sh_ears* e) {
    if (!e) return;
    (void)hipSetDevice(e->device);
    if (e->stream) (void)hipStreamSynchronize(e->stream);
    if (e->mem) (void)hipFree(e->mem);
    if (e->work) (void)hipFree(e->work);
    if (e->host_in) (void)hipHostFree(e->host_in);
    if (e->stream) (void)hipStreamDestroy(e->stream);
    delete e;
}

// one float table in the device layout: [cols / 8][rows_pad][8] of the file's element type
struct tplan {
    std::vector<std::pair<const gg_tensor*, int>> rows;   // (tensor, row)
    const float* dense = nullptr;                          // or a dense fp32 [rows][cols] host matrix
    int n_dense = 0, cols = 0;
    bool f32 = false;
    etab* dst = nullptr;
    size_t bytes() const {
        const size_t nr = dense ? n_dense : rows.size();
        return (nr + 7) / 8 * 8 * cols * (f32 ? 4 : 2);
    }
};

void fill_table(const tplan& t, uint8_t* o) {
    const int nr = t.dense ? t.n_dense : (int)t.rows.size(), rp = (nr + 7) / 8 * 8, K = t.cols;
    memset(o, 0, t.bytes());
    for (int r = 0; r < nr; r++) {
        const uint8_t* src = t.dense ? nullptr
                                     : static_cast<const uint8_t*>(t.rows[r].first->data) +
                                           (size_t)t.rows[r].second * t.rows[r].first->nb[1];
        for (int k = 0; k < K; k++) {
            const size_t at = ((size_t)(k / 8) * rp + r) * 8 + k % 8;
            if (t.f32) {
                const float v = t.dense ? t.dense[(size_t)r * K + k] : reinterpret_cast<const float*>(src)[k];
                memcpy(o + at * 4, &v, 4);
            } else {
                memcpy(o + at * 2, src + (size_t)k * 2, 2);
            }
        }
    }
}

bool is_f32(const gg_tensor* t, int64_t n) {
    return t && t->type == GT_F32 && t->ne[0] * t->ne[1] * t->ne[2] * t->ne[3] == n;
}
bool is_table(const gg_tensor* t, int64_t cols, int64_t rows) {
    return t && (t->type == GT_F16 || t->type == GT_F32) && t->ne[0] == cols && t->ne[1] == rows && t->ne[2] == 1 && t->ne[3] == 1;
}

int run_table(sh_ears* e, int epi, const etab& W, const float* x, int ldx, int P, const float* bias, float* out, int ldo,
              bool xt) {
    etab_args a{};
    a.W = W; a.x = x; a.ldx = ldx; a.P = P; a.bias = bias; a.out = out; a.ldo = ldo; a.xt_out = xt;
    ECHK(launch_etab(epi, a, e->stream));
    return SH_OK;
}
#define RUN(x)                        \
    do {                              \
        const int rc_ = (x);          \
        if (rc_ != SH_OK) return rc_; \
    } while (0)

// the work buffers for a clip of n samples
int ensure_work(sh_ears* e, int n) {
    const sh_ears_shape& I = e->info;
    const geom g = geometry(n, I.n_mel);
    const int C = I.n_ch, E = I.n_embd, Pp = pad16(g.P), Pf = pad16(g.n_fr), P4 = pad16((long)g.T4 * g.F4),
              P8 = pad16((long)g.P * g.F8);
    std::vector<size_t> sz = {
        (size_t)n,                                        // pcm
        (size_t)N_FFT * Pf,                               // fx
        (size_t)N_BIN * Pf,                               // pw
        (size_t)g.n_fr * I.n_mel,                         // mel
        (size_t)C * g.T2 * g.F2,                          // a0
        (size_t)C * P4,                                   // a1
        (size_t)C * P4,                                   // a2
        (size_t)C * P8,                                   // a3
        (size_t)C * P8,                                   // a4
        (size_t)C * g.F8 * Pp,                            // xf
        (size_t)g.P * E,                                  // x
        (size_t)std::max(E, I.n_embd) * Pp,               // h
        (size_t)g.P * e->big_w,                           // big
        (size_t)std::max({I.n_ff, I.n_head * std::max(I.head_dim, 1), E}) * Pp,   // act
        (size_t)e->n_mid * Pp,                            // proj
        (size_t)g.P * I.n_out,                            // out
        (size_t)g.P * std::max(I.head_dim, 2),            // cs (float2 [P][D / 2])
    };
    size_t need = 0;
    for (size_t s : sz) need += (s * 4 + 255) / 256 * 256;
    if (need > e->work_cap) {
        if (e->work) { ECHK(hipStreamSynchronize(e->stream)); ECHK(hipFree(e->work)); e->work = nullptr; e->work_cap = 0; }
        if (hipMalloc((void**)&e->work, need) != hipSuccess) { e->work = nullptr; return set_error(SH_E_NOMEM, "sh_ears_encode: device work buffers"); }
        ECHK(hipMemset(e->work, 0, need));
        e->work_cap = need;
    }
    float** dst[] = {&e->pcm, &e->fx, &e->pw, &e->mel, &e->a0, &e->a1, &e->a2, &e->a3, &e->a4, &e->xf, &e->x, &e->h,
                     &e->big, &e->act, &e->proj, &e->out, reinterpret_cast<float**>(&e->cs)};
    size_t off = 0;
    for (size_t i = 0; i < sz.size(); i++) {
        *dst[i] = reinterpret_cast<float*>(e->work + off);
        off += (sz[i] * 4 + 255) / 256 * 256;
    }
    const size_t host_need = std::max({(size_t)n, (size_t)g.P * I.n_out, (size_t)g.n_fr * I.n_mel, (size_t)g.P * std::max(I.head_dim, 2)});
    if (host_need > e->host_cap) {
        if (e->host_in) { (void)hipHostFree(e->host_in); e->host_in = nullptr; e->host_cap = 0; }
        if (hipHostMalloc((void**)&e->host_in, host_need * 4) != hipSuccess) { e->host_in = nullptr; return set_error(SH_E_NOMEM, "sh_ears_encode: pinned staging"); }
        e->host_cap = host_need;
    }
    return SH_OK;
}

// imi/core/ears.cpp:198-407 on the device; rows end in e->out [P][n_out]
int enqueue_encode(sh_ears* e, int n) {
    const sh_ears_shape& I = e->info;
    const geom g = geometry(n, I.n_mel);
    const int C = I.n_ch, E = I.n_embd, D = I.head_dim, Pp = pad16(g.P), Pf = pad16(g.n_fr), P4 = pad16((long)g.T4 * g.F4),
              P8 = pad16((long)g.P * g.F8);
    hipStream_t s = e->stream;
    // mel (ears.cpp:211-238)
    ECHK(launch_eframes(e->pcm, n, e->hann, N_FFT, HOP, g.n_fr, e->fx, Pf, s));
    RUN(run_table(e, EE_POWER, e->dft, e->fx, Pf, g.n_fr, nullptr, e->pw, Pf, true));
    ECHK(launch_emel(e->pw, Pf, e->fb, e->fb_span, N_BIN, I.n_mel, g.n_fr, e->mel, s));
    // downsampler (ears.cpp:241-296), channel-major
    ECHK(launch_econv0(e->mel, g.n_fr, I.n_mel, e->c0_w, e->c0_b, C, e->a0, s));
    ECHK(launch_edw(e->a0, g.T2, g.F2, g.T2 * g.F2, e->c2_w, e->c2_b, C, e->a1, P4, s));
    RUN(run_table(e, EE_SILU, e->c3, e->a1, P4, g.T4 * g.F4, e->c3_b, e->a2, P4, true));
    ECHK(launch_edw(e->a2, g.T4, g.F4, P4, e->c5_w, e->c5_b, C, e->a3, P8, s));
    RUN(run_table(e, EE_SILU, e->c6, e->a3, P8, g.P * g.F8, e->c6_b, e->a4, P8, true));
    ECHK(launch_eflat(e->a4, P8, C, g.F8, g.P, e->xf, Pp, s));
    RUN(run_table(e, EE_STORE, e->pre, e->xf, Pp, g.P, e->pre_b, e->x, E, false));
    // layers (ears.cpp:302-370)
    for (const elayer& L : e->layers) {
        ECHK(launch_enorm(e->x, L.ln1, E, g.P, e->eps, e->h, Pp, s));
        const int ld = L.in.rows;
        RUN(run_table(e, EE_STORE, L.in, e->h, Pp, g.P, nullptr, e->big, ld, false));
        if (!L.attn) {
            ECHK(launch_econv(e->big, ld, L.conv_w, E, I.d_conv, g.P, e->act, Pp, s));
        } else {
            ECHK(launch_eqk(e->big, ld, I.n_head, I.n_head_kv, D, L.q_norm, L.k_norm, e->cs, g.P, e->eps, s));
            ECHK(launch_eattn(e->big, ld, I.n_head, I.n_head_kv, D, I.window, g.P, e->act, Pp, s));
        }
        RUN(run_table(e, EE_ADD, L.out, e->act, Pp, g.P, nullptr, e->x, E, false));
        ECHK(launch_enorm(e->x, L.ln2, E, g.P, e->eps, e->h, Pp, s));
        RUN(run_table(e, EE_GLU, L.gate_up, e->h, Pp, g.P, nullptr, e->act, Pp, true));
        RUN(run_table(e, EE_ADD, L.down, e->act, Pp, g.P, nullptr, e->x, E, false));
    }
    // last norm, LayerNorm, projector (ears.cpp:372-403)
    ECHK(launch_efinal(e->x, e->post_ln, e->ln_w, e->ln_b, E, g.P, e->eps, e->h, Pp, s));
    RUN(run_table(e, EE_GELU, e->mlp1, e->h, Pp, g.P, e->mlp1_b, e->proj, Pp, true));
    RUN(run_table(e, EE_STORE, e->mlp3, e->proj, Pp, g.P, e->mlp3_b, e->out, I.n_out, false));
    return SH_OK;
}

}  // namespace

extern "C" {

int sh_ears_load(int device, const char* path, sh_ears** out) {   // imi/core/ears.cpp:40-138
    if (!path || !out) return set_error(SH_E_ARG, "sh_ears_load: bad argument");
    *out = nullptr;
    ECHK(hipSetDevice(device));
    gg_file f;
    if (!f.load(path)) return set_error(SH_E_FILE, "sh_ears_load: " + f.error);
    const gg_tensor* pre_w = f.get("a.pre_encode.out.weight", false);
    if (!pre_w) return set_error(SH_E_FILE, std::string("sh_ears_load: ") + path + " has no ears");
    sh_ears_shape I{};
    I.n_mel = (int)f.key_i("clip.audio.num_mel_bins", 128);
    I.window = (int)f.key_i("clip.audio.window_size", 32);
    I.n_head = (int)f.key_i("clip.audio.attention.head_count", 8);
    const float eps = f.key_f("clip.audio.attention.layer_norm_epsilon", 1e-5f);
    const gg_tensor* c0 = f.get("a.conv1d.0.weight", false);
    if (!c0) return set_error(SH_E_FILE, "sh_ears_load: no a.conv1d.0.weight");
    const int C = (int)c0->ne[3];
    I.n_ch = C;
    const char* convs[] = {"a.conv1d.0", "a.conv1d.2", "a.conv1d.5"};
    for (const char* nm : convs) {
        const gg_tensor *w = f.get(std::string(nm) + ".weight", false), *b = f.get(std::string(nm) + ".bias", false);
        if (!w || !b || w->type != GT_F32 || w->ne[0] != 3 || w->ne[1] != 3 || w->ne[2] != 1 || w->ne[3] != C || !is_f32(b, C))
            return set_error(SH_E_SHAPE, std::string("sh_ears_load: ") + nm + " must be F32 3 x 3 taps of " + std::to_string(C) + " channels");
    }
    for (const char* nm : {"a.conv1d.3", "a.conv1d.6"}) {
        const gg_tensor *w = f.get(std::string(nm) + ".weight", false), *b = f.get(std::string(nm) + ".bias", false);
        if (!w || !b || !is_f32(w, (int64_t)C * C) || w->ne[2] != C || w->ne[3] != C || !is_f32(b, C))
            return set_error(SH_E_SHAPE, std::string("sh_ears_load: ") + nm + " must be an F32 C x C pointwise table");
    }
    if (I.n_mel < 8 || I.n_mel % 8 || C < 1 || C % 8)
        return set_error(SH_E_SHAPE, "sh_ears_load: n_mel must be a multiple of 8 and the channels a multiple of 8");
    const int E = (int)pre_w->ne[1];
    I.n_embd = E;
    const gg_tensor* pre_b = f.get("a.pre_encode.out.bias", false);
    if (!is_table(pre_w, (int64_t)C * I.n_mel / 8, E) || !is_f32(pre_b, E) || E % 32 || E > 4096)
        return set_error(SH_E_SHAPE, "sh_ears_load: pre_encode.out must be an F16/F32 table of n_ch * n_mel / 8 columns, "
                                     "n_embd a multiple of 32 up to 4096");
    if (I.window < 1 || I.window > EA_MAX_WIN) return set_error(SH_E_SHAPE, "sh_ears_load: window must be 1 to 64");

    std::vector<tplan> tabs;
    struct vec { const float* src; std::vector<float> host; int n; const float** dst; };
    std::vector<vec> vecs;
    auto v_of = [&](const gg_tensor* t, int n, const float** dst) { vecs.push_back({static_cast<const float*>(t->data), {}, n, dst}); };
    std::vector<elayer> layers;
    int n_attn = 0;
    for (int il = 0;; il++) {
        if (!f.get("a.blk." + std::to_string(il) + ".ln1.weight", false)) break;
        layers.emplace_back();
    }
    if (layers.empty()) return set_error(SH_E_FILE, "sh_ears_load: no layers");
    int big_w = 3 * E;
    for (size_t il = 0; il < layers.size(); il++) {
        const std::string p = "a.blk." + std::to_string(il) + ".";
        elayer& L = layers[il];
        const gg_tensor *l1 = f.get(p + "ln1.weight", false), *l2 = f.get(p + "ln2.weight", false);
        const gg_tensor *fg = f.get(p + "ffn_gate.weight", false), *fu = f.get(p + "ffn_up.weight", false),
                        *fd = f.get(p + "ffn_down.weight", false);
        if (!is_f32(l1, E) || !is_f32(l2, E)) return set_error(SH_E_SHAPE, "sh_ears_load: layer norms must be F32 of n_embd");
        if (!fg || !fu || !fd) return set_error(SH_E_FILE, "sh_ears_load: FFN tables missing in layer " + std::to_string(il));
        if (il == 0) I.n_ff = (int)fg->ne[1];
        if (!is_table(fg, E, I.n_ff) || !is_table(fu, E, I.n_ff) || fu->type != fg->type || !is_table(fd, I.n_ff, E) ||
            I.n_ff % 8 || I.n_ff < 8)
            return set_error(SH_E_SHAPE, "sh_ears_load: FFN tables must be F16/F32, n_ff a multiple of 8, the same in every layer");
        v_of(l1, E, &L.ln1);
        v_of(l2, E, &L.ln2);
        if (const gg_tensor* dw = f.get(p + "conv_dw.weight", false)) {
            const gg_tensor *w1 = f.get(p + "conv_pw1.weight", false), *w2 = f.get(p + "conv_pw2.weight", false);
            const int K = (int)dw->ne[0];
            if (I.d_conv == 0) I.d_conv = K;
            if (dw->type != GT_F32 || dw->ne[1] != E || K != I.d_conv || K < 1 || K > 16 || !is_table(w1, E, 3 * E) ||
                !is_table(w2, E, E))
                return set_error(SH_E_SHAPE, "sh_ears_load: conv layer must have F32 taps (1 to 16, the same in every layer) "
                                             "and F16/F32 pw1 (3 n_embd rows) / pw2 tables");
            vec tv{nullptr, std::vector<float>((size_t)K * E), K * E, &L.conv_w};   // [channel][tap] -> [tap][channel]
            for (int ee = 0; ee < E; ee++)
                for (int k = 0; k < K; k++) tv.host[(size_t)k * E + ee] = static_cast<const float*>(dw->data)[(size_t)ee * K + k];
            vecs.push_back(std::move(tv));
            tplan a{}; a.cols = E; a.f32 = w1->type == GT_F32; a.dst = &L.in;
            for (int r = 0; r < 3 * E; r++) a.rows.push_back({w1, r});
            tabs.push_back(std::move(a));
            tplan b{}; b.cols = E; b.f32 = w2->type == GT_F32; b.dst = &L.out;
            for (int r = 0; r < E; r++) b.rows.push_back({w2, r});
            tabs.push_back(std::move(b));
        } else {
            L.attn = true;
            const gg_tensor *qn = f.get(p + "attn_q_norm.weight", false), *kn = f.get(p + "attn_k_norm.weight", false);
            const gg_tensor *q = f.get(p + "attn_q.weight", false), *k = f.get(p + "attn_k.weight", false),
                            *v = f.get(p + "attn_v.weight", false), *o = f.get(p + "attn_out.weight", false);
            if (!qn || !kn || !q || !k || !v || !o) return set_error(SH_E_FILE, "sh_ears_load: attention tensors missing in layer " + std::to_string(il));
            const int D = (int)qn->ne[0];
            if (n_attn == 0) { I.head_dim = D; I.n_head_kv = D > 0 ? (int)(k->ne[1] / D) : 0; }
            const int H = I.n_head, Hk = I.n_head_kv;
            if (D != I.head_dim || D % 32 || D < 32 || D > EA_MAX_D || Hk < 1 || H < 1 || H % Hk || !is_f32(qn, D) ||
                !is_f32(kn, D) || !is_table(q, E, (int64_t)H * D) || !is_table(k, E, (int64_t)Hk * D) ||
                !is_table(v, E, (int64_t)Hk * D) || !is_table(o, (int64_t)H * D, E) || q->type != k->type || k->type != v->type)
                return set_error(SH_E_SHAPE, "sh_ears_load: attention shapes not supported (head_dim a multiple of 32 up to "
                                             "128, head_count a multiple of the kv heads, F16/F32 tables)");
            v_of(qn, D, &L.q_norm);
            v_of(kn, D, &L.k_norm);
            tplan a{}; a.cols = E; a.f32 = q->type == GT_F32; a.dst = &L.in;   // q | k | v stacked (ears.cpp:121)
            for (const gg_tensor* t : {q, k, v}) for (int r = 0; r < (int)t->ne[1]; r++) a.rows.push_back({t, r});
            tabs.push_back(std::move(a));
            tplan b{}; b.cols = H * D; b.f32 = o->type == GT_F32; b.dst = &L.out;
            for (int r = 0; r < E; r++) b.rows.push_back({o, r});
            tabs.push_back(std::move(b));
            big_w = std::max(big_w, (H + 2 * Hk) * D);
            n_attn++;
        }
        tplan gu{}; gu.cols = E; gu.f32 = fg->type == GT_F32; gu.dst = &L.gate_up;   // gate / up by 8-row group (ears.cpp:128-130)
        for (int t = 0; t < I.n_ff; t += 8) {
            for (int r = t; r < t + 8; r++) gu.rows.push_back({fg, r});
            for (int r = t; r < t + 8; r++) gu.rows.push_back({fu, r});
        }
        tabs.push_back(std::move(gu));
        tplan dn{}; dn.cols = I.n_ff; dn.f32 = fd->type == GT_F32; dn.dst = &L.down;
        for (int r = 0; r < E; r++) dn.rows.push_back({fd, r});
        tabs.push_back(std::move(dn));
    }
    if (n_attn == 0) { I.head_dim = 0; I.n_head_kv = 0; }
    I.n_layer = (int)layers.size();
    I.n_attn = n_attn;
    const gg_tensor *post = f.get("a.post_ln.weight", false), *lw = f.get("mm.a.mlp.0.weight", false),
                    *lb = f.get("mm.a.mlp.0.bias", false), *m1 = f.get("mm.a.mlp.1.weight", false),
                    *m1b = f.get("mm.a.mlp.1.bias", false), *m3 = f.get("mm.a.mlp.3.weight", false),
                    *m3b = f.get("mm.a.mlp.3.bias", false);
    if (!is_f32(post, E) || !is_f32(lw, E) || !is_f32(lb, E) || !m1 || !m3)
        return set_error(SH_E_SHAPE, "sh_ears_load: post_ln / projector LayerNorm must be F32 of n_embd");
    const int n_mid = (int)m1->ne[1];
    I.n_out = (int)m3->ne[1];
    if (!is_table(m1, E, n_mid) || !is_f32(m1b, n_mid) || !is_table(m3, n_mid, I.n_out) || !is_f32(m3b, I.n_out) ||
        n_mid % 8 || n_mid < 8 || I.n_out < 1)
        return set_error(SH_E_SHAPE, "sh_ears_load: projector tables must be F16/F32 (mlp.1 n_embd -> a multiple of 8, "
                                     "mlp.3 -> n_out)");

    auto* e = new sh_ears;
    e->device = device;
    e->eps = eps;
    e->n_mid = n_mid;
    I.n_mid = n_mid;
    e->big_w = big_w;
    e->layers = std::move(layers);
    // the mel front end as imi builds it (ears.cpp:44-80)
    std::vector<float> hann(N_FFT), dftm((size_t)2 * N_BIN * N_FFT), fbm((size_t)I.n_mel * N_BIN, 0.0f);
    for (int i = 0; i < N_FFT; i++) hann[i] = (float)(0.5 * (1.0 - cos(2.0 * M_PI * i / N_FFT)));
    for (int b = 0; b < N_BIN; b++)
        for (int k = 0; k < N_FFT; k++) {
            const double a = 2.0 * M_PI * (double)((size_t)b * k % N_FFT) / N_FFT;
            dftm[(size_t)(2 * b) * N_FFT + k] = (float)cos(a);
            dftm[(size_t)(2 * b + 1) * N_FFT + k] = (float)-sin(a);
        }
    {
        const double sr = 16000, lin = 3.0 / 200, min_log_mel = 15.0, step = log(6.4) / 27;
        auto hz2mel = [&](double hz) { return hz < 1000 ? hz * lin : min_log_mel + log(hz / 1000) / step; };
        auto mel2hz = [&](double m) { return m < min_log_mel ? m / lin : 1000 * exp((m - min_log_mel) * step); };
        const double lo = hz2mel(0), hi = hz2mel(sr / 2);
        std::vector<double> pts(I.n_mel + 2);
        for (int i = 0; i < I.n_mel + 2; i++) pts[i] = mel2hz(lo + (hi - lo) * i / (I.n_mel + 1));
        for (int m = 0; m < I.n_mel; m++) {
            const double fl = pts[m], fc = pts[m + 1], fr = pts[m + 2], en = 2.0 / (fr - fl);
            for (int b = 0; b < N_BIN; b++) {
                const double hz = b * sr / N_FFT;
                double w = 0;
                if (hz >= fl && hz <= fc) w = (hz - fl) / (fc - fl);
                else if (hz > fc && hz <= fr) w = (fr - hz) / (fr - fc);
                fbm[(size_t)m * N_BIN + b] = (float)(w * en);
            }
        }
    }
    auto taps9 = [&](const char* nm, const float** dst) {   // [ch][3][3] -> [kh * 3 + kw][ch] (ears.cpp:15-22)
        const float* d = static_cast<const float*>(f.get(nm)->data);
        vec tv{nullptr, std::vector<float>((size_t)9 * C), 9 * C, dst};
        for (int c = 0; c < C; c++) for (int j = 0; j < 9; j++) tv.host[(size_t)j * C + c] = d[(size_t)c * 9 + j];
        vecs.push_back(std::move(tv));
    };
    vecs.push_back({nullptr, hann, N_FFT, &e->hann});
    vecs.push_back({nullptr, fbm, I.n_mel * N_BIN, &e->fb});
    {
        vec sp{nullptr, std::vector<float>((size_t)2 * I.n_mel), 2 * I.n_mel, reinterpret_cast<const float**>(&e->fb_span)};
        for (int m = 0; m < I.n_mel; m++) {
            int lo = 0, hi = 0;
            for (int b = 0; b < N_BIN; b++)
                if (fbm[(size_t)m * N_BIN + b] != 0.0f) { if (hi == 0) lo = b; hi = b + 1; }
            const int32_t v[2] = {lo, hi};
            memcpy(&sp.host[(size_t)2 * m], v, 8);
        }
        vecs.push_back(std::move(sp));
    }
    taps9("a.conv1d.0.weight", &e->c0_w); v_of(f.get("a.conv1d.0.bias"), C, &e->c0_b);
    taps9("a.conv1d.2.weight", &e->c2_w); v_of(f.get("a.conv1d.2.bias"), C, &e->c2_b);
    taps9("a.conv1d.5.weight", &e->c5_w); v_of(f.get("a.conv1d.5.bias"), C, &e->c5_b);
    v_of(f.get("a.conv1d.3.bias"), C, &e->c3_b);
    v_of(f.get("a.conv1d.6.bias"), C, &e->c6_b);
    v_of(pre_b, E, &e->pre_b);
    v_of(post, E, &e->post_ln);
    v_of(lw, E, &e->ln_w);
    v_of(lb, E, &e->ln_b);
    v_of(m1b, n_mid, &e->mlp1_b);
    v_of(m3b, I.n_out, &e->mlp3_b);
    {
        tplan t{}; t.dense = dftm.data(); t.n_dense = 2 * N_BIN; t.cols = N_FFT; t.f32 = true; t.dst = &e->dft; tabs.push_back(t);
    }
    for (auto [nm, dst] : {std::pair<const char*, etab*>{"a.conv1d.3.weight", &e->c3}, {"a.conv1d.6.weight", &e->c6}}) {
        tplan t{}; t.dense = static_cast<const float*>(f.get(nm)->data); t.n_dense = C; t.cols = C; t.f32 = true; t.dst = dst;
        tabs.push_back(t);
    }
    auto whole = [&](const gg_tensor* t, etab* dst) {
        tplan p{}; p.cols = (int)t->ne[0]; p.f32 = t->type == GT_F32; p.dst = dst;
        for (int r = 0; r < (int)t->ne[1]; r++) p.rows.push_back({t, r});
        tabs.push_back(std::move(p));
    };
    whole(pre_w, &e->pre);
    whole(m1, &e->mlp1);
    whole(m3, &e->mlp3);

    size_t need = 0, tbytes = 0;
    for (const tplan& t : tabs) { need += (t.bytes() + 255) / 256 * 256; tbytes += t.bytes(); }
    for (const vec& v : vecs) need += ((size_t)v.n * 4 + 255) / 256 * 256;
    I.table_bytes = (long long)tbytes;
    e->info = I;
    if (hipStreamCreate(&e->stream) != hipSuccess) { release(e); return set_error(SH_E_HIP, "sh_ears_load: stream"); }
    if (hipMalloc((void**)&e->mem, need) != hipSuccess) { e->mem = nullptr; release(e); return set_error(SH_E_NOMEM, "sh_ears_load: device memory"); }
    std::vector<uint8_t> host(need, 0);
    size_t off = 0;
    for (const tplan& t : tabs) {
        fill_table(t, host.data() + off);
        const int nr = t.dense ? t.n_dense : (int)t.rows.size();
        t.dst->w = e->mem + off;
        t.dst->rows = nr;
        t.dst->rows_pad = (nr + 7) / 8 * 8;
        t.dst->cols = t.cols;
        t.dst->f32 = t.f32;
        off += (t.bytes() + 255) / 256 * 256;
    }
    for (const vec& v : vecs) {
        memcpy(host.data() + off, v.src ? v.src : v.host.data(), (size_t)v.n * 4);
        *v.dst = reinterpret_cast<const float*>(e->mem + off);
        off += ((size_t)v.n * 4 + 255) / 256 * 256;
    }
    if (hipMemcpy(e->mem, host.data(), need, hipMemcpyHostToDevice) != hipSuccess) {
        release(e);
        return set_error(SH_E_HIP, "sh_ears_load: upload");
    }
    *out = e;
    return SH_OK;
}

int sh_ears_free(sh_ears* e) {
    if (!e) return set_error(SH_E_ARG, "sh_ears_free: null");
    release(e);
    return SH_OK;
}

int sh_ears_info(const sh_ears* e, sh_ears_shape* out) {
    if (!e || !out) return set_error(SH_E_ARG, "sh_ears_info: bad argument");
    *out = e->info;
    return SH_OK;
}

int sh_ears_positions(const sh_ears* e, int n, int* n_pos, int* n_frames) {
    if (!e || n < 0) return set_error(SH_E_ARG, "sh_ears_positions: bad argument");
    const geom g = geometry(n, e->info.n_mel);
    if (n_pos) *n_pos = g.P;
    if (n_frames) *n_frames = g.n_fr;
    return SH_OK;
}

int sh_ears_encode(sh_ears* e, const float* pcm, int n, float* out, int* n_pos) {   // ears.cpp:198-407
    if (!e || !out || n < 1 || !pcm) return set_error(SH_E_ARG, "sh_ears_encode: bad argument (n_samples >= 1)");
    if (n > (1 << 28)) return set_error(SH_E_ARG, "sh_ears_encode: clip too long");
    ECHK(hipSetDevice(e->device));
    RUN(ensure_work(e, n));
    const sh_ears_shape& I = e->info;
    const geom g = geometry(n, I.n_mel);
    // rope rows of positions 0 .. P - 1 as imi's rope forms them (ears.cpp:23-31): th = position, times
    // theta^(-2/D) per pair, with the C library's powf / cosf / sinf
    if (I.head_dim > 0) {
        const int D = I.head_dim;
        const float scale = powf(e->theta, -2.0f / (float)D);
        float2* cs = reinterpret_cast<float2*>(e->host_in);
        for (int p = 0; p < g.P; p++) {
            float th = (float)p;
            for (int i = 0; i < D / 2; i++) {
                cs[(size_t)p * (D / 2) + i] = make_float2(cosf(th), sinf(th));
                th *= scale;
            }
        }
        ECHK(hipMemcpyAsync(e->cs, e->host_in, (size_t)g.P * (D / 2) * sizeof(float2), hipMemcpyHostToDevice, e->stream));
        ECHK(hipStreamSynchronize(e->stream));
    }
    memcpy(e->host_in, pcm, (size_t)n * 4);
    ECHK(hipMemcpyAsync(e->pcm, e->host_in, (size_t)n * 4, hipMemcpyHostToDevice, e->stream));
    RUN(enqueue_encode(e, n));
    ECHK(hipMemcpyAsync(e->host_in, e->out, (size_t)g.P * I.n_out * 4, hipMemcpyDeviceToHost, e->stream));
    ECHK(hipStreamSynchronize(e->stream));
    memcpy(out, e->host_in, (size_t)g.P * I.n_out * 4);
    e->last_frames = g.n_fr;
    if (n_pos) *n_pos = g.P;
    return SH_OK;
}

int sh_ears_mel(const sh_ears* e, float* mel, int cap_frames, int* n_frames) {
    if (!e || (!mel && !n_frames) || cap_frames < 0) return set_error(SH_E_ARG, "sh_ears_mel: bad argument");
    if (!e->mel || e->last_frames == 0) return set_error(SH_E_STATE, "sh_ears_mel: nothing encoded yet");
    if (n_frames) *n_frames = e->last_frames;
    if (!mel) return SH_OK;   // the frame count only
    if (e->last_frames > cap_frames)
        return set_error(SH_E_ARG, "sh_ears_mel: the last encode has " + std::to_string(e->last_frames) +
                                       " frames, the buffer holds " + std::to_string(cap_frames));
    ECHK(hipSetDevice(e->device));
    ECHK(hipMemcpy(mel, e->mel, (size_t)e->last_frames * e->info.n_mel * 4, hipMemcpyDeviceToHost));
    return SH_OK;
}

}  // extern "C"
