// ORACLE — test infrastructure only (see imi_cpu.h). Restatement of imi's codec decoder (imi/core/codec.{h,cpp}):
// 12 codes -> FSQ level rows -> quantizer projection -> in_proj -> 6 positions -> LFM layers (short conv with carried
// memory, gated attention over the last 30 positions with carried keys/values) -> norm -> out_proj -> 641 log
// magnitudes + 641 phases per position -> inverse FFT (1280 points, mixed radix) -> periodic Hann overlap-add.
// One thread: the codec is small next to the brain (imi runs it on the shared team, imi/core/codec.cpp:114-119).
//
// Arithmetic: as the source is written, with the contraction GCC applies to it under imi's flags (-march=native,
// gnu++17 and so -ffp-contract=fast): `s += a * b` is fmaf(a, b, s); `a * b - c * d` and `a * b + c * d` fuse the
// first product, fmaf(a, b, -(c * d)) / fmaf(a, b, c * d) (the convention this oracle follows for imi's rope,
// imi/core/seoul.cpp:19-28); `s = b[o]; s += w * q` is one chain from the bias. Complex products follow the same
// rule: (a + bi)(c + di) = fmaf(a, c, -(b * d)) + fmaf(a, d, b * c) i. The float64 restatement of
// imi/ref/codec_exact.py (oracle/exact.py) pins these numbers; imi's own binary is not buildable here.
#include "imi_cpu.h"

#include <algorithm>
#include <cmath>
#include <cstdio>
#include <cstring>
#include <string>
#include <vector>

namespace orc {
namespace {

const float* f32(const gtensor* t) { return t ? (const float*)t->data : nullptr; }
inline float silu(float x) { return x / (1.0f + expf(-x)); }

struct cplx { float re, im; };
inline cplx cmul(cplx a, cplx b) { return {fmaf(a.re, b.re, -(a.im * b.im)), fmaf(a.re, b.im, a.im * b.re)}; }
inline cplx cadd(cplx a, cplx b) { return {a.re + b.re, a.im + b.im}; }
inline cplx csub(cplx a, cplx b) { return {a.re - b.re, a.im - b.im}; }

// imi/core/codec.cpp:25-39: inverse DFT, halving while the size is even, a direct sum at the odd base
void ifft_rec(const cplx* in, int n, int stride, cplx* out, const cplx* tw, int tws) {
    if (n % 2) {
        for (int k = 0; k < n; k++) {
            cplx s = {0.0f, 0.0f};
            for (int j = 0; j < n; j++) s = cadd(s, cmul(in[(size_t)j * stride], tw[(size_t)((j * k) % n) * tws]));
            out[k] = s;
        }
        return;
    }
    const int h = n / 2;
    ifft_rec(in, h, 2 * stride, out, tw, 2 * tws);
    ifft_rec(in + stride, h, 2 * stride, out + h, tw, 2 * tws);
    for (int k = 0; k < h; k++) {
        const cplx e = out[k], o = cmul(out[k + h], tw[(size_t)k * tws]);
        out[k] = cadd(e, o);
        out[k + h] = csub(e, o);
    }
}

void transpose(const float* a, int P, int K, int lda, float* t) {
    for (int p = 0; p < P; p++) for (int k = 0; k < K; k++) t[(size_t)k * P + p] = a[(size_t)p * lda + k];
}

}  // namespace

struct codec {
    struct layer {
        const float *ln1, *ln2, *post1, *post2;
        q8gtab gate_up, down, pw1, pw2, qkv, o;
        std::vector<float> conv_w;        // [tap][channel]
        const float* gate_w = nullptr;    // [n_head][n_embd]
        const float *q_norm = nullptr, *k_norm = nullptr;
        bool conv = false;
    };
    gfile f;
    std::vector<layer> layers;
    const float *lvl = nullptr, *qo_w = nullptr, *qo_b = nullptr, *in_b = nullptr, *out_b = nullptr, *out_norm = nullptr;
    q8gtab in_proj, out_proj;
    int n_codes = 0, n_lvl = 0, n_cb = 12, n_embd = 0, n_ff = 0, n_head = 0, n_head_kv = 0, head_dim = 0, d_conv = 0, n_q = 0;
    int n_fs = 6, window = 30, n_fft = 1280, hop = 320, n_bins = 641;
    float eps = 1e-5f, theta = 1e6f;
    // carried state
    std::vector<std::vector<float>> conv_state, k_win, v_win;
    int pos = 0;
    std::vector<float> ola, wsum, hann;
    std::vector<cplx> tw;
    int pad_left = 0;
    // work
    std::vector<float> x, h, xt, big, y, act, spec;

    bool load(const std::string& path);
    void reset();
    void frame(const int32_t* codes, std::vector<float>& pcm);
    void flush(std::vector<float>& pcm);
    void run(const int32_t* codes);
    void istft(const float* lp, std::vector<float>& pcm);
};

bool codec::load(const std::string& path) {   // imi/core/codec.cpp:41-108
    if (!f.open(path)) return false;
    const std::string g = "a.gen.wav.";
    const gtensor* cb = f.get(g + "quant.first.codebook.weight");
    const gtensor* ip = f.get(g + "tfm.in_proj.weight");
    const gtensor* op = f.get(g + "tfm.out_proj.weight");
    if (!cb || !ip || !op) { fprintf(stderr, "oracle: codec tensor missing\n"); return false; }
    lvl = f32(cb); n_lvl = (int)cb->ne[0]; n_codes = (int)cb->ne[1];
    qo_w = f32(f.get(g + "quant.first.out_proj.weight")); qo_b = f32(f.get(g + "quant.first.out_proj.bias"));
    in_b = f32(f.get(g + "tfm.in_proj.bias")); out_b = f32(f.get(g + "tfm.out_proj.bias"));
    out_norm = f32(f.get(g + "tfm.output_norm.weight"));
    auto rows_of = [](std::vector<const uint8_t*>& o, const gtensor* t, int r0, int n) {
        for (int r = r0; r < r0 + n; r++) o.push_back(t->data + (size_t)r * t->row_bytes);
    };
    auto whole = [&](q8gtab& dst, std::vector<const gtensor*> parts) {
        std::vector<const uint8_t*> o;
        for (auto* p : parts) { if (!p || p->type != T_Q8_0) return false; rows_of(o, p, 0, (int)p->ne[1]); }
        return q8g_build(dst, o, (int)parts[0]->ne[0]);
    };
    n_embd = (int)ip->ne[1];
    n_q = (int)ip->ne[0];
    bool ok = whole(in_proj, {ip}) && whole(out_proj, {op});
    n_bins = (int)op->ne[1] / 2;
    for (int il = 0;; il++) {
        const std::string p = g + "tfm.blk." + std::to_string(il) + ".";
        if (!f.get(p + "ln1.weight")) break;
        layer L;
        L.ln1 = f32(f.get(p + "ln1.weight")); L.ln2 = f32(f.get(p + "ln2.weight"));
        L.post1 = f32(f.get(p + "attn_post_norm.weight")); L.post2 = f32(f.get(p + "ffn_post_norm.weight"));
        if (const gtensor* cw = f.get(p + "conv_dw.weight")) {
            L.conv = true;
            const int K = (int)cw->ne[0], C = (int)cw->ne[1];
            d_conv = K - 1;
            L.conv_w.resize((size_t)K * C);
            for (int e = 0; e < C; e++) for (int k = 0; k < K; k++) L.conv_w[(size_t)k * C + e] = f32(cw)[(size_t)e * K + k];
            ok &= whole(L.pw1, {f.get(p + "conv_pw1.weight")}) && whole(L.pw2, {f.get(p + "conv_pw2.weight")});
        } else {
            L.q_norm = f32(f.get(p + "attn_q_norm.weight")); L.k_norm = f32(f.get(p + "attn_k_norm.weight"));
            const gtensor *q = f.get(p + "attn_q.weight"), *k = f.get(p + "attn_k.weight"), *gw = f.get(p + "attn_gate.weight");
            if (!q || !k || !gw || !L.q_norm || gw->type != T_F32) return false;
            head_dim = (int)f.get(p + "attn_q_norm.weight")->ne[0];
            n_head = (int)(q->ne[1] / head_dim); n_head_kv = (int)(k->ne[1] / head_dim);
            ok &= whole(L.qkv, {q, k, f.get(p + "attn_v.weight")}) && whole(L.o, {f.get(p + "attn_out.weight")});
            L.gate_w = f32(gw);
        }
        const gtensor *fg = f.get(p + "ffn_gate.weight"), *fu = f.get(p + "ffn_up.weight");
        if (!fg || !fu) return false;
        n_ff = (int)fg->ne[1];
        std::vector<const uint8_t*> o;
        for (int t = 0; t < n_ff; t += 8) { rows_of(o, fg, t, 8); rows_of(o, fu, t, 8); }
        ok &= q8g_build(L.gate_up, o, (int)fg->ne[0]) && whole(L.down, {f.get(p + "ffn_down.weight")});
        layers.push_back(std::move(L));
    }
    if (!ok) { fprintf(stderr, "oracle: a codec table is not 8-bit\n"); return false; }
    const int P = n_fs, E = n_embd, wide = std::max({3 * E, n_ff, 2 * n_bins + 8, n_head * head_dim + 2 * n_head_kv * head_dim});
    x.resize((size_t)P * E); h.resize((size_t)P * wide); xt.resize((size_t)P * wide);
    big.resize((size_t)P * wide); y.resize((size_t)P * E); act.resize((size_t)P * wide); spec.resize((size_t)P * 2 * n_bins);
    hann.resize(n_fft); tw.resize(n_fft);
    for (int i = 0; i < n_fft; i++) {   // codec.cpp:101-104
        hann[i] = 0.5f * (1.0f - cosf(2.0f * (float)M_PI * i / n_fft));
        const float a = 2.0f * (float)M_PI * i / n_fft;
        tw[i] = {cosf(a), sinf(a)};   // std::polar(1.0f, a)
    }
    reset();
    return true;
}

void codec::reset() {   // codec.cpp:110-119
    pos = 0;
    const int kvd = n_head_kv * head_dim;
    conv_state.assign(layers.size(), {}); k_win.assign(layers.size(), {}); v_win.assign(layers.size(), {});
    for (size_t il = 0; il < layers.size(); il++) {
        if (layers[il].conv) conv_state[il].assign((size_t)d_conv * n_embd, 0.0f);
        else { k_win[il].assign((size_t)(window - 1) * kvd, 0.0f); v_win[il].assign((size_t)(window - 1) * kvd, 0.0f); }
    }
    ola.assign(n_fft, 0.0f); wsum.assign(n_fft, 0.0f);
    pad_left = (n_fft - hop) / 2;
}

void codec::frame(const int32_t* codes, std::vector<float>& pcm) {   // codec.cpp:121-127
    run(codes);
    pos += n_fs;
    for (int p = 0; p < n_fs; p++) istft(spec.data() + (size_t)p * 2 * n_bins, pcm);
}

// codec.cpp:129-252 with one thread
void codec::run(const int32_t* codes) {
    const int E = n_embd, P = n_fs, D = head_dim, kvd = n_head_kv * D, grp = n_head / n_head_kv, W1 = window - 1;
    auto table = [&](const q8gtab& W, int C, const float* in, float* o, int ldo, const float* bias) {
        std::vector<float> tmp((size_t)C * 8);
        for (int gg = 0; gg < W.rows_pad / 8; gg++) {
            q8g_group(W, in, C, gg, tmp.data());
            for (int p = 0; p < C; p++) for (int r = 0; r < 8 && 8 * gg + r < W.rows; r++)
                o[(size_t)p * ldo + 8 * gg + r] = tmp[8 * p + r] + (bias ? bias[8 * gg + r] : 0.0f);
        }
    };
    {   // codec.cpp:147-159: the frame's vector
        const int nq = n_cb * n_lvl;
        std::vector<float> q((size_t)nq), v((size_t)n_q);
        for (int i = 0; i < n_cb; i++) for (int l = 0; l < n_lvl; l++) q[(size_t)i * n_lvl + l] = lvl[(size_t)codes[i] * n_lvl + l];
        for (int o = 0; o < n_q; o++) { float s = qo_b[o]; for (int i = 0; i < nq; i++) s = fmaf(qo_w[(size_t)o * nq + i], q[i], s); v[o] = s; }
        table(in_proj, 1, v.data(), x.data(), E, in_b);
        for (int p = 1; p < P; p++) memcpy(x.data() + (size_t)p * E, x.data(), (size_t)E * sizeof(float));
    }
    for (size_t il = 0; il < layers.size(); il++) {
        const layer& L = layers[il];
        for (int p = 0; p < P; p++) norm_mul(x.data() + (size_t)p * E, L.ln1, h.data() + (size_t)p * E, E, eps);
        transpose(h.data(), P, E, E, xt.data());
        if (L.conv) {   // codec.cpp:163-192
            table(L.pw1, P, xt.data(), big.data(), 3 * E, nullptr);
            std::vector<float> bx((size_t)P * E), u((size_t)P * E);
            for (int p = 0; p < P; p++) for (int e = 0; e < E; e++) bx[(size_t)p * E + e] = big[(size_t)p * 3 * E + e] * big[(size_t)p * 3 * E + 2 * E + e];
            const float* st = conv_state[il].data();
            for (int p = 0; p < P; p++) {
                float* up = u.data() + (size_t)p * E;
                for (int e = 0; e < E; e++) up[e] = 0.0f;
                for (int k = 0; k <= d_conv; k++) {
                    const int t = p + k;
                    const float* src = t < d_conv ? st + (size_t)t * E : bx.data() + (size_t)(t - d_conv) * E;
                    const float* wk = L.conv_w.data() + (size_t)k * E;
                    for (int e = 0; e < E; e++) up[e] = fmaf(src[e], wk[e], up[e]);
                }
                const float* cc = big.data() + (size_t)p * 3 * E + E;
                for (int e = 0; e < E; e++) up[e] *= cc[e];
            }
            transpose(u.data(), P, E, E, xt.data());
            table(L.pw2, P, xt.data(), y.data(), E, nullptr);
            std::vector<float> all((size_t)(d_conv + P) * E);
            memcpy(all.data(), st, (size_t)d_conv * E * sizeof(float));
            memcpy(all.data() + (size_t)d_conv * E, bx.data(), (size_t)P * E * sizeof(float));
            memcpy(conv_state[il].data(), all.data() + (size_t)P * E, (size_t)d_conv * E * sizeof(float));
        } else {   // codec.cpp:193-236
            const int nq = n_head * D, nr = nq + 2 * kvd;
            table(L.qkv, P, xt.data(), big.data(), nr, nullptr);
            std::vector<float> K((size_t)(W1 + P) * kvd), V((size_t)(W1 + P) * kvd);
            memcpy(K.data(), k_win[il].data(), (size_t)W1 * kvd * sizeof(float));
            memcpy(V.data(), v_win[il].data(), (size_t)W1 * kvd * sizeof(float));
            for (int p = 0; p < P; p++) {
                const float* r = big.data() + (size_t)p * nr;
                for (int g = 0; g < n_head_kv; g++) {
                    float* kk = K.data() + (size_t)(W1 + p) * kvd + g * D;
                    norm_mul(r + nq + g * D, L.k_norm, kk, D, eps);
                    rope(kk, D, pos + p, theta, nullptr);
                }
                memcpy(V.data() + (size_t)(W1 + p) * kvd, r + nq + kvd, (size_t)kvd * sizeof(float));
            }
            for (int hh = 0; hh < n_head; hh++) {
                const int kv = hh / grp;
                for (int p = 0; p < P; p++) {
                    float q[128], sc[64];
                    norm_mul(big.data() + (size_t)p * nr + hh * D, L.q_norm, q, D, eps);
                    rope(q, D, pos + p, theta, nullptr);
                    float mx = -INFINITY;
                    for (int j = p; j <= p + W1; j++) {
                        if (pos - W1 + j < 0) { sc[j - p] = -INFINITY; continue; }
                        float s = 0.0f;
                        const float* kk = K.data() + (size_t)j * kvd + kv * D;
                        for (int i = 0; i < D; i++) s = fmaf(q[i], kk[i], s);
                        sc[j - p] = s / sqrtf((float)D);
                        mx = std::max(mx, sc[j - p]);
                    }
                    float sum = 0.0f;
                    for (int j = 0; j <= W1; j++) { sc[j] = sc[j] == -INFINITY ? 0.0f : expf(sc[j] - mx); sum += sc[j]; }
                    float gs = 0.0f;
                    const float *gw = L.gate_w + (size_t)hh * E, *hp = h.data() + (size_t)p * E;
                    for (int e = 0; e < E; e++) gs = fmaf(gw[e], hp[e], gs);
                    const float gate = 1.0f / (1.0f + expf(-gs));
                    float* o = act.data() + (size_t)p * nq + hh * D;
                    for (int i = 0; i < D; i++) {
                        float a = 0.0f;
                        for (int j = 0; j <= W1; j++) a = fmaf(sc[j], V[(size_t)(p + j) * kvd + kv * D + i], a);
                        o[i] = a / sum * gate;
                    }
                }
            }
            memcpy(k_win[il].data(), K.data() + (size_t)P * kvd, (size_t)W1 * kvd * sizeof(float));
            memcpy(v_win[il].data(), V.data() + (size_t)P * kvd, (size_t)W1 * kvd * sizeof(float));
            transpose(act.data(), P, nq, nq, xt.data());
            table(L.o, P, xt.data(), y.data(), E, nullptr);
        }
        for (int p = 0; p < P; p++) norm_mul_add(y.data() + (size_t)p * E, L.post1, x.data() + (size_t)p * E, E, eps);
        for (int p = 0; p < P; p++) norm_mul(x.data() + (size_t)p * E, L.ln2, h.data() + (size_t)p * E, E, eps);
        transpose(h.data(), P, E, E, xt.data());
        {   // codec.cpp:239-247: (gate, up) group pairs -> silu(gate) * up
            std::vector<float> a((size_t)P * 8), b((size_t)P * 8);
            for (int g = 0; g < L.gate_up.rows_pad / 8; g += 2) {
                q8g_group(L.gate_up, xt.data(), P, g, a.data());
                q8g_group(L.gate_up, xt.data(), P, g + 1, b.data());
                for (int p = 0; p < P; p++) for (int r = 0; r < 8; r++) act[(size_t)p * n_ff + 4 * g + r] = silu(a[8 * p + r]) * b[8 * p + r];
            }
        }
        transpose(act.data(), P, n_ff, n_ff, xt.data());
        table(L.down, P, xt.data(), y.data(), E, nullptr);
        for (int p = 0; p < P; p++) norm_mul_add(y.data() + (size_t)p * E, L.post2, x.data() + (size_t)p * E, E, eps);
    }
    for (int p = 0; p < P; p++) norm_mul(x.data() + (size_t)p * E, out_norm, h.data() + (size_t)p * E, E, eps);
    transpose(h.data(), P, E, E, xt.data());
    table(out_proj, P, xt.data(), spec.data(), 2 * n_bins, out_b);
}

// codec.cpp:254-269: one STFT frame
void codec::istft(const float* lp, std::vector<float>& pcm) {
    std::vector<cplx> X(n_fft, cplx{0.0f, 0.0f}), xo(n_fft);
    for (int k = 0; k < n_bins; k++) {   // std::polar(expf(lp[k]), lp[n_bins + k])
        const float r = expf(lp[k]), a = lp[n_bins + k];
        X[k] = {r * cosf(a), r * sinf(a)};
    }
    for (int k = 1; k < n_bins - 1; k++) X[n_fft - k] = {X[k].re, -X[k].im};
    ifft_rec(X.data(), n_fft, 1, xo.data(), tw.data(), 1);
    for (int j = 0; j < n_fft; j++) {
        ola[j] = fmaf(xo[j].re / (float)n_fft, hann[j], ola[j]);
        wsum[j] = fmaf(hann[j], hann[j], wsum[j]);
    }
    for (int i = 0; i < hop; i++) {
        const float s = wsum[i] > 1e-8f ? ola[i] / wsum[i] : ola[i];
        if (pad_left > 0) pad_left--; else pcm.push_back(s);
    }
    std::copy(ola.begin() + hop, ola.end(), ola.begin()); std::fill(ola.end() - hop, ola.end(), 0.0f);
    std::copy(wsum.begin() + hop, wsum.end(), wsum.begin()); std::fill(wsum.end() - hop, wsum.end(), 0.0f);
}

void codec::flush(std::vector<float>& pcm) {   // codec.cpp:271-277
    const int tail = n_fft - hop, trim = (n_fft - hop) / 2;
    for (int i = 0; i < tail - trim; i++) pcm.push_back(wsum[i] > 1e-8f ? ola[i] / wsum[i] : ola[i]);
    reset();
}

}  // namespace orc

using namespace orc;
extern "C" {

void* orc_codec_load(const char* path) {
    auto* c = new codec;
    if (!c->load(path)) { delete c; return nullptr; }
    return c;
}
void orc_codec_free(void* h) { delete (codec*)h; }
// n_embd, n_ff, n_head, n_head_kv, head_dim, d_conv, n_layer, n_bins, n_lvl, n_q, pos, n_codes
void orc_codec_info(void* h, int* o) {
    auto* c = (codec*)h;
    const int v[12] = {c->n_embd, c->n_ff, c->n_head, c->n_head_kv, c->head_dim, c->d_conv, (int)c->layers.size(),
                       c->n_bins, c->n_lvl, c->n_q, c->pos, c->n_codes};
    memcpy(o, v, sizeof(v));
}
void orc_codec_reset(void* h) { ((codec*)h)->reset(); }
// one frame of 12 codes: its samples into pcm (capacity 6 * hop), returns how many; spec (nullable) gets the
// frame's [6][2 * n_bins] log magnitudes and phases
int orc_codec_frame(void* h, const int32_t* codes, float* pcm, float* spec) {
    auto* c = (codec*)h;
    std::vector<float> out;
    c->frame(codes, out);
    memcpy(pcm, out.data(), out.size() * sizeof(float));
    if (spec) memcpy(spec, c->spec.data(), c->spec.size() * sizeof(float));
    return (int)out.size();
}
int orc_codec_flush(void* h, float* pcm) {
    auto* c = (codec*)h;
    std::vector<float> out;
    c->flush(out);
    memcpy(pcm, out.data(), out.size() * sizeof(float));
    return (int)out.size();
}
// the inverse DFT alone (n a power of two times an odd factor): x = sum_k X_k e^{2 pi i jk / n}, no 1/n
void orc_ifft(const float* re, const float* im, int n, float* ore, float* oim) {
    std::vector<cplx> in(n), out(n), tw(n);
    for (int i = 0; i < n; i++) {
        in[i] = {re[i], im[i]};
        const float a = 2.0f * (float)M_PI * i / n;
        tw[i] = {cosf(a), sinf(a)};
    }
    ifft_rec(in.data(), n, 1, out.data(), tw.data(), 1);
    for (int i = 0; i < n; i++) { ore[i] = out[i].re; oim[i] = out[i].im; }
}

}  // extern "C"
