// ORACLE — test infrastructure only (see imi_cpu.h). Restatement of imi's ears, the audio encoder
// (imi/core/ears.{h,cpp}): 16 kHz samples -> 128 mel bands every 10 ms (Hann frames through the DFT as a 12-input
// float table, power, Slaney filters summed in double, log10) -> three stride-2 3x3 convolutions (pointwise tables
// between) -> pre_encode projection -> causal LFM layers (pre-norm; short conv, or attention over the last `window`
// positions) -> last norm, LayerNorm, 768 -> 2048, GELU (erf), 2048 -> 2048.
//
// Arithmetic as the source is written under imi's flags (-ffp-contract=fast, see imi_cpu_codec.cpp): `s += a * b`
// is fmaf(a, b, s) (in double for the mel sums); `a * a + b * b` fuses the first product. The float tables follow
// imi_wg_group12 (imi/core/tables.cpp:522-556): per row and input one chain acc = fma(w, x, acc) over the columns in
// order, from zero; weights F16 (exact in fp32) or F32. Pinned to the float64 restatement of imi/ref/ears_exact.py
// (oracle/exact.py) by tests/test_oracle_ears.py.
#include "imi_cpu.h"

#include <algorithm>
#include <chrono>
#include <cmath>
#include <cstdio>
#include <cstring>
#include <string>
#include <vector>

namespace orc {
namespace {

inline float silu_e(float x) { return x / (1.0f + expf(-x)); }                              // ears.cpp:32
inline float gelu_erf(float x) { return 0.5f * x * (1.0f + erff(x * 0.70710678118654752f)); }   // ears.cpp:33

// imi_wg (imi/core/tables.h:84-95): rows padded to 8, [row group][col][8], F16 bits or F32
struct wgtab {
    int rows = 0, cols = 0, rows_pad = 0;
    bool f32 = false;
    std::vector<uint16_t> h;
    std::vector<float> f;
};
template <class G> void wg_fill(wgtab& W, int rows, int cols, bool is32, G get) {   // tables.cpp:481-493
    W.rows = rows; W.cols = cols; W.rows_pad = (rows + 7) / 8 * 8; W.f32 = is32;
    const size_t n = (size_t)W.rows_pad * cols;
    if (is32) W.f.assign(n, 0.0f); else W.h.assign(n, 0);
    for (int r = 0; r < rows; r++) for (int k = 0; k < cols; k++) {
        const size_t at = ((size_t)(r / 8) * cols + k) * 8 + r % 8;
        if (is32) W.f[at] = get(r, k, 0.0f); else W.h[at] = (uint16_t)get(r, k, 0);
    }
}
// rows of one or more tensors stacked (tables.cpp:495-512): all F16 or all F32, same column count
bool wg_build(wgtab& W, const std::vector<std::pair<const gtensor*, int>>& rows) {
    if (rows.empty() || !rows[0].first) return false;
    const gtensor* t0 = rows[0].first;
    const int c = (int)t0->ne[0];
    for (const auto& p : rows) if (!p.first || p.first->type != t0->type || p.first->ne[0] != c) return false;
    if (t0->type != T_F16 && t0->type != T_F32) return false;
    auto row = [&](int i) { return rows[i].first->data + (size_t)rows[i].second * rows[i].first->row_bytes; };
    if (t0->type == T_F16)
        wg_fill(W, (int)rows.size(), c, false, [&](int i, int k, int) { return (int)((const uint16_t*)row(i))[k]; });
    else
        wg_fill(W, (int)rows.size(), c, true, [&](int i, int k, float) { return ((const float*)row(i))[k]; });
    return true;
}
bool wg_build(wgtab& W, const gtensor* t) {
    if (!t || t->ne[2] != 1 || t->ne[3] != 1) return false;
    std::vector<std::pair<const gtensor*, int>> r;
    for (int i = 0; i < (int)t->ne[1]; i++) r.push_back({t, i});
    return wg_build(W, r);
}
void wg_build(wgtab& W, const float* m, int r, int c) {   // tables.cpp:518-521
    wg_fill(W, r, c, true, [&](int i, int k, float) { return m[(size_t)i * c + k]; });
}

// imi_wg_group12 (tables.cpp:522-556): group g's 8 rows times 12 inputs xt [cols][12] -> out [12][8]
void wg_group12(const wgtab& W, const float* xt, int g, float* out) {
    __m256 a[12];
    for (int c = 0; c < 12; c++) a[c] = _mm256_setzero_ps();
    for (int k = 0; k < W.cols; k++) {
        const size_t at = ((size_t)g * W.cols + k) * 8;
        const __m256 wv = W.f32 ? _mm256_loadu_ps(W.f.data() + at)
                                : _mm256_cvtph_ps(_mm_loadu_si128((const __m128i*)(W.h.data() + at)));
        const float* xk = xt + (size_t)k * 12;
        for (int c = 0; c < 12; c++) a[c] = _mm256_fmadd_ps(wv, _mm256_broadcast_ss(xk + c), a[c]);
    }
    for (int c = 0; c < 12; c++) _mm256_storeu_ps(out + 8 * c, a[c]);
}

const float* f32p(const gtensor* t) { return t ? (const float*)t->data : nullptr; }
std::vector<float> copy_f32(const gtensor* t) {
    if (!t || t->type != T_F32) return {};
    const float* d = f32p(t);
    return std::vector<float>(d, d + t->ne[0] * t->ne[1] * t->ne[2] * t->ne[3]);
}
std::vector<float> taps9(const gtensor* t) {   // ears.cpp:15-22: [ch][3][3] -> [kh*3+kw][ch]
    const int C = (int)t->ne[3];
    const float* d = f32p(t);
    std::vector<float> o((size_t)9 * C);
    for (int c = 0; c < C; c++) for (int j = 0; j < 9; j++) o[(size_t)j * C + c] = d[(size_t)c * 9 + j];
    return o;
}

}  // namespace

struct ears {
    struct layer {
        bool attn = false;
        std::vector<float> ln1, ln2, conv_w, q_norm, k_norm;
        wgtab in, out, gate_up, down;
    };
    gfile f;
    std::vector<layer> layers;
    std::vector<float> c0_w, c0_b, c2_w, c2_b, c3_b, c5_w, c5_b, c6_b;
    wgtab dft, c3, c6, pre, mlp1, mlp3;
    std::vector<float> hann, fb, pre_b, post_ln, ln_w, ln_b, mlp1_b, mlp3_b;
    int n_mel = 128, n_bin = 201, n_fft = 400, hop = 160, n_ch = 256, n_embd = 768, n_ff = 0, n_head = 0, n_head_kv = 0,
        head_dim = 0, window = 32, n_out = 0, d_conv = 3;
    float eps = 1e-5f, rope_theta = 1e6f;
    team tm;
    std::vector<float> xt, xres, buf, buf2, last_mel;
    double t_mel = 0, t_down = 0, t_layers = 0, t_proj = 0;

    void par(int n, const std::function<void(int)>& fn) {   // ears.cpp:140-144: units handed out by a counter
        if (n <= 0) return;
        std::atomic<int> ctr{0};
        tm.run([&](int) { for (int u = ctr.fetch_add(1); u < n; u = ctr.fetch_add(1)) fn(u); });
    }
    bool load(const std::string& path, int threads);
    int encode(const float* pcm, int n, std::vector<float>& out);
    void pack(const float* a, int P, int K, int lda, float* o);
    void table(const wgtab& W, const float* x, int P, float* out, int ldo, const float* bias, bool add);
    void table_glu(const wgtab& W, const float* x, int P, float* out);
};

bool ears::load(const std::string& path, int threads) {   // imi/core/ears.cpp:40-138
    if (!f.open(path)) return false;
    if (!f.get("a.pre_encode.out.weight")) { fprintf(stderr, "oracle: %s has no ears\n", path.c_str()); return false; }
    bool ok = true;
    hann.resize(n_fft);
    for (int i = 0; i < n_fft; i++) hann[i] = (float)(0.5 * (1.0 - cos(2.0 * M_PI * i / n_fft)));
    n_bin = n_fft / 2 + 1;
    {
        std::vector<float> m((size_t)2 * n_bin * n_fft);
        for (int b = 0; b < n_bin; b++) for (int k = 0; k < n_fft; k++) {
            const double a = 2.0 * M_PI * (double)((size_t)b * k % n_fft) / n_fft;
            m[(size_t)(2 * b) * n_fft + k] = (float)cos(a);
            m[(size_t)(2 * b + 1) * n_fft + k] = (float)-sin(a);
        }
        wg_build(dft, m.data(), 2 * n_bin, n_fft);
    }
    n_mel = (int)f.key_i("clip.audio.num_mel_bins", 128);
    {   // Slaney mel filters (ears.cpp:62-80)
        const double sr = 16000, lin = 3.0 / 200, min_log_mel = 15.0, step = log(6.4) / 27;
        auto hz2mel = [&](double hz) { return hz < 1000 ? hz * lin : min_log_mel + log(hz / 1000) / step; };
        auto mel2hz = [&](double m) { return m < min_log_mel ? m / lin : 1000 * exp((m - min_log_mel) * step); };
        const double lo = hz2mel(0), hi = hz2mel(sr / 2);
        std::vector<double> pts(n_mel + 2);
        for (int i = 0; i < n_mel + 2; i++) pts[i] = mel2hz(lo + (hi - lo) * i / (n_mel + 1));
        fb.assign((size_t)n_mel * n_bin, 0.0f);
        for (int m = 0; m < n_mel; m++) {
            const double fl = pts[m], fc = pts[m + 1], fr = pts[m + 2], en = 2.0 / (fr - fl);
            for (int b = 0; b < n_bin; b++) {
                const double hz = b * sr / n_fft;
                double w = 0;
                if (hz >= fl && hz <= fc) w = (hz - fl) / (fc - fl);
                else if (hz > fc && hz <= fr) w = (fr - hz) / (fr - fc);
                fb[(size_t)m * n_bin + b] = (float)(w * en);
            }
        }
    }
    const gtensor* c0 = f.get("a.conv1d.0.weight");
    for (const char* nm : {"a.conv1d.0.weight", "a.conv1d.0.bias", "a.conv1d.2.weight", "a.conv1d.2.bias", "a.conv1d.3.weight",
                           "a.conv1d.3.bias", "a.conv1d.5.weight", "a.conv1d.5.bias", "a.conv1d.6.weight", "a.conv1d.6.bias"}) {
        const gtensor* t = f.get(nm);
        if (!t || t->type != T_F32) { fprintf(stderr, "oracle: %s missing or not F32\n", nm); return false; }
    }
    n_ch = (int)c0->ne[3];
    c0_w = taps9(c0);                          c0_b = copy_f32(f.get("a.conv1d.0.bias"));
    c2_w = taps9(f.get("a.conv1d.2.weight"));  c2_b = copy_f32(f.get("a.conv1d.2.bias"));
    c5_w = taps9(f.get("a.conv1d.5.weight"));  c5_b = copy_f32(f.get("a.conv1d.5.bias"));
    wg_build(c3, f32p(f.get("a.conv1d.3.weight")), n_ch, n_ch); c3_b = copy_f32(f.get("a.conv1d.3.bias"));
    wg_build(c6, f32p(f.get("a.conv1d.6.weight")), n_ch, n_ch); c6_b = copy_f32(f.get("a.conv1d.6.bias"));
    ok &= wg_build(pre, f.get("a.pre_encode.out.weight")); pre_b = copy_f32(f.get("a.pre_encode.out.bias"));
    n_embd = pre.rows;
    if (pre.cols != n_ch * n_mel / 8) { fprintf(stderr, "oracle: unexpected downsampler width %d\n", pre.cols); return false; }
    window = (int)f.key_i("clip.audio.window_size", 32);
    n_head = (int)f.key_i("clip.audio.attention.head_count", 8);
    eps = f.key_f("clip.audio.attention.layer_norm_epsilon", 1e-5f);
    auto rows = [](std::vector<std::pair<const gtensor*, int>>& o, const gtensor* t, int r0, int n) {
        for (int r = r0; r < r0 + n; r++) o.push_back({t, r});
    };
    for (int il = 0;; il++) {
        const std::string p = "a.blk." + std::to_string(il) + ".";
        if (!f.get(p + "ln1.weight")) break;
        layer L;
        L.ln1 = copy_f32(f.get(p + "ln1.weight")); L.ln2 = copy_f32(f.get(p + "ln2.weight"));
        std::vector<std::pair<const gtensor*, int>> in;
        if (const gtensor* dw = f.get(p + "conv_dw.weight")) {
            d_conv = (int)dw->ne[0];
            L.conv_w.resize((size_t)d_conv * n_embd);
            const float* d = f32p(dw);
            for (int e = 0; e < n_embd; e++) for (int k = 0; k < d_conv; k++) L.conv_w[(size_t)k * n_embd + e] = d[(size_t)e * d_conv + k];
            const gtensor* pw1 = f.get(p + "conv_pw1.weight");
            if (!pw1) return false;
            rows(in, pw1, 0, (int)pw1->ne[1]);
            ok &= wg_build(L.out, f.get(p + "conv_pw2.weight"));
        } else {
            L.attn = true;
            L.q_norm = copy_f32(f.get(p + "attn_q_norm.weight")); L.k_norm = copy_f32(f.get(p + "attn_k_norm.weight"));
            head_dim = (int)L.q_norm.size();
            const gtensor *q = f.get(p + "attn_q.weight"), *k = f.get(p + "attn_k.weight"), *v = f.get(p + "attn_v.weight");
            if (!q || !k || !v || head_dim == 0) return false;
            n_head_kv = (int)(k->ne[1] / head_dim);
            rows(in, q, 0, (int)q->ne[1]); rows(in, k, 0, (int)k->ne[1]); rows(in, v, 0, (int)v->ne[1]);
            ok &= wg_build(L.out, f.get(p + "attn_out.weight"));
        }
        ok &= wg_build(L.in, in);
        const gtensor *fg = f.get(p + "ffn_gate.weight"), *fu = f.get(p + "ffn_up.weight");
        if (!fg || !fu) return false;
        n_ff = (int)fg->ne[1];
        std::vector<std::pair<const gtensor*, int>> gu;
        for (int t = 0; t < n_ff; t += 8) { rows(gu, fg, t, 8); rows(gu, fu, t, 8); }
        ok &= wg_build(L.gate_up, gu);
        ok &= wg_build(L.down, f.get(p + "ffn_down.weight"));
        layers.push_back(std::move(L));
    }
    post_ln = copy_f32(f.get("a.post_ln.weight"));
    ln_w = copy_f32(f.get("mm.a.mlp.0.weight")); ln_b = copy_f32(f.get("mm.a.mlp.0.bias"));
    ok &= wg_build(mlp1, f.get("mm.a.mlp.1.weight")); mlp1_b = copy_f32(f.get("mm.a.mlp.1.bias"));
    ok &= wg_build(mlp3, f.get("mm.a.mlp.3.weight")); mlp3_b = copy_f32(f.get("mm.a.mlp.3.bias"));
    n_out = mlp3.rows;
    if (!ok || layers.empty() || n_ff % 8 || n_embd % 32 || head_dim % 32) {
        fprintf(stderr, "oracle: an ears table has an unexpected type or shape\n");
        return false;
    }
    tm.start(threads);
    return true;
}

void ears::pack(const float* a, int P, int K, int lda, float* o) {   // ears.cpp:146-155: 12-position chunks [K][12]
    par((P + 11) / 12, [&](int ch) {
        float* d = o + (size_t)ch * K * 12;
        for (int j = 0; j < 12; j++) {
            const int p = ch * 12 + j;
            if (p < P) { const float* r = a + (size_t)p * lda; for (int k = 0; k < K; k++) d[(size_t)k * 12 + j] = r[k]; }
            else for (int k = 0; k < K; k++) d[(size_t)k * 12 + j] = 0.0f;
        }
    });
}

// ears.cpp:158-180: out[p][row] (+)= acc + (bias or 0)
void ears::table(const wgtab& W, const float* x, int P, float* out, int ldo, const float* bias, bool add) {
    const int ng = W.rows_pad / 8, nch = (P + 11) / 12;
    par(ng * nch, [&](int u) {
        const int g = u % ng, ch = u / ng;
        float tmp[96];
        wg_group12(W, x + (size_t)ch * W.cols * 12, g, tmp);
        const int nr = std::min(8, W.rows - 8 * g);
        for (int j = 0; j < 12 && ch * 12 + j < P; j++) {
            float* o = out + (size_t)(ch * 12 + j) * ldo + 8 * g;
            for (int r = 0; r < nr; r++) {
                const float v = tmp[8 * j + r] + (bias ? bias[8 * g + r] : 0.0f);
                o[r] = add ? o[r] + v : v;
            }
        }
    });
}

// ears.cpp:182-196: (gate, up) group pairs -> out[p][8q + r] = silu(gate) * up
void ears::table_glu(const wgtab& W, const float* x, int P, float* out) {
    const int npair = W.rows_pad / 16, half = W.rows / 2, nch = (P + 11) / 12;
    par(npair * nch, [&](int u) {
        const int q = u % npair, ch = u / npair;
        float a[96], b[96];
        const float* xc = x + (size_t)ch * W.cols * 12;
        wg_group12(W, xc, 2 * q, a);
        wg_group12(W, xc, 2 * q + 1, b);
        for (int j = 0; j < 12 && ch * 12 + j < P; j++)
            for (int r = 0; r < 8; r++) out[(size_t)(ch * 12 + j) * half + 8 * q + r] = silu_e(a[8 * j + r]) * b[8 * j + r];
    });
}

int ears::encode(const float* pcm, int n, std::vector<float>& out) {   // imi/core/ears.cpp:198-407
    using clk = std::chrono::steady_clock;
    auto secs = [](clk::time_point a) { return std::chrono::duration<double>(clk::now() - a).count(); };
    auto t0 = clk::now();
    const int n_pad = n <= n_fft ? n_fft : n + (hop - (n - n_fft) % hop) % hop;
    const int n_fr = (n_pad - n_fft) / hop + 1;
    const int T2 = (n_fr + 1) / 2, F2 = n_mel / 2, T4 = (T2 + 1) / 2, F4 = F2 / 2, P = (T4 + 1) / 2, F8 = F4 / 2;
    const int C = n_ch, E = n_embd;
    auto ch12 = [](int v) { return (size_t)(v + 11) / 12 * 12; };
    xt.resize(std::max({ch12(T4 * F4) * C, ch12(P * F8) * C, ch12(P) * pre.cols, ch12(P) * n_ff, ch12(P) * n_out,
                        ch12(P) * mlp1.rows}));
    buf.resize(std::max({(size_t)T2 * F2 * C, (size_t)T4 * F4 * C, (size_t)P * layers[0].in.rows, (size_t)P * 3 * E,
                         (size_t)P * n_ff, (size_t)P * n_out, (size_t)P * mlp1.rows}));
    buf2.resize((size_t)T4 * F4 * C);
    xres.resize((size_t)P * E);

    // mel (ears.cpp:211-238)
    last_mel.assign((size_t)n_fr * n_mel, 0.0f);
    float* mel = last_mel.data();
    par((n_fr + 11) / 12, [&](int ch) {
        std::vector<float> fx((size_t)n_fft * 12), pw((size_t)12 * n_bin);
        for (int j = 0; j < 12; j++) {
            const int fr = ch * 12 + j;
            for (int k = 0; k < n_fft; k++) {
                const int i = fr * hop + k;
                fx[(size_t)k * 12 + j] = fr < n_fr && i < n ? hann[k] * pcm[i] : 0.0f;
            }
        }
        float tmp[96];
        for (int g = 0; g < dft.rows_pad / 8; g++) {
            wg_group12(dft, fx.data(), g, tmp);
            for (int j = 0; j < 12; j++) for (int r = 0; r < 8; r += 2) {
                const int b = 4 * g + r / 2;
                if (b < n_bin) pw[(size_t)j * n_bin + b] = fmaf(tmp[8 * j + r], tmp[8 * j + r], tmp[8 * j + r + 1] * tmp[8 * j + r + 1]);
            }
        }
        for (int j = 0; j < 12; j++) {
            const int fr = ch * 12 + j;
            if (fr >= n_fr) break;
            for (int m = 0; m < n_mel; m++) {
                double s = 0;
                const float* w = fb.data() + (size_t)m * n_bin;
                for (int b = 0; b < n_bin; b++) s = std::fma((double)w[b], (double)pw[(size_t)j * n_bin + b], s);
                mel[(size_t)fr * n_mel + m] = (float)((log10(std::max(s, 1e-12)) + 4.0) / 4.0);
            }
        }
    });
    t_mel += secs(t0); t0 = clk::now();

    // downsampler (ears.cpp:241-296), [time][freq][ch]
    float* a0 = buf.data();
    par(T2, [&](int t) {
        for (int fq = 0; fq < F2; fq++) {
            float* o = a0 + ((size_t)t * F2 + fq) * C;
            for (int c = 0; c < C; c++) o[c] = c0_b[c];
            for (int kh = 0; kh < 3; kh++) for (int kw = 0; kw < 3; kw++) {
                const int ti = 2 * t + kw - 1, fi = 2 * fq + kh - 1;
                if (ti < 0 || ti >= n_fr || fi < 0 || fi >= n_mel) continue;
                const float v = mel[(size_t)ti * n_mel + fi], *w = c0_w.data() + (size_t)(kh * 3 + kw) * C;
                for (int c = 0; c < C; c++) o[c] = fmaf(v, w[c], o[c]);
            }
            for (int c = 0; c < C; c++) o[c] = silu_e(o[c]);
        }
    });
    auto dw = [&](const float* in, int Ti, int Fi, const std::vector<float>& w, const std::vector<float>& b, float* o_) {
        const int To = (Ti + 1) / 2, Fo = Fi / 2;
        par(To, [&](int t) {
            for (int fq = 0; fq < Fo; fq++) {
                float* o = o_ + ((size_t)t * Fo + fq) * C;
                for (int c = 0; c < C; c++) o[c] = b[c];
                for (int kh = 0; kh < 3; kh++) for (int kw = 0; kw < 3; kw++) {
                    const int ti = 2 * t + kw - 1, fi = 2 * fq + kh - 1;
                    if (ti < 0 || ti >= Ti || fi < 0 || fi >= Fi) continue;
                    const float *v = in + ((size_t)ti * Fi + fi) * C, *ww = w.data() + (size_t)(kh * 3 + kw) * C;
                    for (int c = 0; c < C; c++) o[c] = fmaf(v[c], ww[c], o[c]);
                }
            }
        });
    };
    auto silu_all = [&](float* a, size_t cnt) {
        const size_t blk = 1 << 14;
        par((int)((cnt + blk - 1) / blk), [&](int u) {
            for (size_t i = (size_t)u * blk; i < std::min(cnt, (size_t)(u + 1) * blk); i++) a[i] = silu_e(a[i]);
        });
    };
    dw(a0, T2, F2, c2_w, c2_b, buf2.data());
    pack(buf2.data(), T4 * F4, C, C, xt.data());
    table(c3, xt.data(), T4 * F4, buf.data(), C, c3_b.data(), false);
    silu_all(buf.data(), (size_t)T4 * F4 * C);
    dw(buf.data(), T4, F4, c5_w, c5_b, buf2.data());
    pack(buf2.data(), P * F8, C, C, xt.data());
    table(c6, xt.data(), P * F8, buf.data(), C, c6_b.data(), false);
    silu_all(buf.data(), (size_t)P * F8 * C);
    {   // [P][F8][C] -> feature c * F8 + f
        const float* a3 = buf.data();
        const int K = C * F8;
        par((P + 11) / 12, [&](int ch) {
            float* d = xt.data() + (size_t)ch * K * 12;
            for (int j = 0; j < 12; j++) {
                const int p = ch * 12 + j;
                for (int c = 0; c < C; c++) for (int fq = 0; fq < F8; fq++)
                    d[(size_t)(c * F8 + fq) * 12 + j] = p < P ? a3[((size_t)p * F8 + fq) * C + c] : 0.0f;
            }
        });
    }
    float* x = xres.data();
    table(pre, xt.data(), P, x, E, pre_b.data(), false);
    t_down += secs(t0); t0 = clk::now();

    // layers (ears.cpp:302-370)
    auto norm_pack = [&](const std::vector<float>& w) {
        par((P + 11) / 12, [&](int ch) {
            float* d = xt.data() + (size_t)ch * E * 12;
            std::vector<float> h(E);
            for (int j = 0; j < 12; j++) {
                const int p = ch * 12 + j;
                if (p < P) norm_mul(x + (size_t)p * E, w.data(), h.data(), E, eps); else std::fill(h.begin(), h.end(), 0.0f);
                for (int k = 0; k < E; k++) d[(size_t)k * 12 + j] = h[k];
            }
        });
    };
    const int D = head_dim;
    for (const layer& L : layers) {
        norm_pack(L.ln1);
        const int ld = L.in.rows;
        table(L.in, xt.data(), P, buf.data(), ld, nullptr, false);
        if (!L.attn) {
            par((P + 11) / 12, [&](int ch) {
                float* d = xt.data() + (size_t)ch * E * 12;
                for (int j = 0; j < 12; j++) {
                    const int p = ch * 12 + j;
                    if (p >= P) { for (int e = 0; e < E; e++) d[(size_t)e * 12 + j] = 0.0f; continue; }
                    for (int e = 0; e < E; e++) {
                        float co = 0;
                        for (int k = 0; k < d_conv; k++) {
                            const int t = p - (d_conv - 1) + k;
                            if (t < 0) continue;
                            const float* r = buf.data() + (size_t)t * ld;
                            co = fmaf(L.conv_w[(size_t)k * E + e], r[e] * r[2 * E + e], co);
                        }
                        d[(size_t)e * 12 + j] = buf[(size_t)p * ld + E + e] * co;
                    }
                }
            });
        } else {
            const int Hq = n_head * D, Hk = n_head_kv * D, grp = n_head / n_head_kv;
            par(P, [&](int p) {
                float* r = buf.data() + (size_t)p * ld;
                for (int h = 0; h < n_head; h++) {
                    norm_mul(r + h * D, L.q_norm.data(), r + h * D, D, eps);
                    rope(r + h * D, D, p, rope_theta, nullptr);
                }
                for (int h = 0; h < n_head_kv; h++) {
                    float* k = r + Hq + h * D;
                    norm_mul(k, L.k_norm.data(), k, D, eps);
                    rope(k, D, p, rope_theta, nullptr);
                }
            });
            const float scale = 1.0f / sqrtf((float)D);
            par((P + 11) / 12, [&](int ch) {
                float* d = xt.data() + (size_t)ch * Hq * 12;
                std::vector<float> sc(window), o(D);
                for (int j = 0; j < 12; j++) {
                    const int p = ch * 12 + j;
                    for (int hh = 0; hh < n_head; hh++) {
                        if (p >= P) { for (int i = 0; i < D; i++) d[(size_t)(hh * D + i) * 12 + j] = 0.0f; continue; }
                        const int kv = hh / grp, s0 = std::max(0, p - window + 1), nk = p - s0 + 1;
                        const float* q = buf.data() + (size_t)p * ld + hh * D;
                        float mx = -INFINITY;
                        for (int t = 0; t < nk; t++) {
                            const float* k = buf.data() + (size_t)(s0 + t) * ld + Hq + kv * D;
                            float s = 0;
                            for (int i = 0; i < D; i++) s = fmaf(q[i], k[i], s);
                            sc[t] = s * scale;
                            mx = std::max(mx, sc[t]);
                        }
                        float sum = 0;
                        for (int t = 0; t < nk; t++) { sc[t] = expf(sc[t] - mx); sum += sc[t]; }
                        std::fill(o.begin(), o.end(), 0.0f);
                        for (int t = 0; t < nk; t++) {
                            const float* v = buf.data() + (size_t)(s0 + t) * ld + Hq + Hk + kv * D;
                            for (int i = 0; i < D; i++) o[i] = fmaf(sc[t], v[i], o[i]);
                        }
                        for (int i = 0; i < D; i++) d[(size_t)(hh * D + i) * 12 + j] = o[i] / sum;
                    }
                }
            });
        }
        table(L.out, xt.data(), P, x, E, nullptr, true);
        norm_pack(L.ln2);
        table_glu(L.gate_up, xt.data(), P, buf.data());
        pack(buf.data(), P, n_ff, n_ff, xt.data());
        table(L.down, xt.data(), P, x, E, nullptr, true);
    }
    t_layers += secs(t0); t0 = clk::now();

    // last norm, LayerNorm, projector (ears.cpp:372-403)
    par((P + 11) / 12, [&](int ch) {
        float* d = xt.data() + (size_t)ch * E * 12;
        std::vector<float> h(E);
        for (int j = 0; j < 12; j++) {
            const int p = ch * 12 + j;
            if (p < P) {
                norm_mul(x + (size_t)p * E, post_ln.data(), h.data(), E, eps);
                double mu = 0, var = 0;
                for (int k = 0; k < E; k++) mu += h[k];
                mu /= E;
                for (int k = 0; k < E; k++) var = std::fma(h[k] - mu, h[k] - mu, var);
                const float inv = (float)(1.0 / sqrt(var / E + 1e-5));
                for (int k = 0; k < E; k++) h[k] = fmaf((float)(h[k] - mu) * inv, ln_w[k], ln_b[k]);
            } else std::fill(h.begin(), h.end(), 0.0f);
            for (int k = 0; k < E; k++) d[(size_t)k * 12 + j] = h[k];
        }
    });
    table(mlp1, xt.data(), P, buf.data(), mlp1.rows, mlp1_b.data(), false);
    {
        const size_t cnt = (size_t)P * mlp1.rows, blk = 1 << 14;
        float* a = buf.data();
        par((int)((cnt + blk - 1) / blk), [&](int u) {
            for (size_t i = (size_t)u * blk; i < std::min(cnt, (size_t)(u + 1) * blk); i++) a[i] = gelu_erf(a[i]);
        });
    }
    pack(buf.data(), P, mlp1.rows, mlp1.rows, xt.data());
    out.resize((size_t)P * n_out);
    table(mlp3, xt.data(), P, out.data(), n_out, mlp3_b.data(), false);
    t_proj += secs(t0);
    return P;
}

}  // namespace orc

using orc::ears;

extern "C" {
void* orc_ears_load(const char* path, int threads) {
    auto* e = new ears;
    if (!e->load(path, threads)) { delete e; return nullptr; }
    return e;
}
void orc_ears_free(void* h) { delete (ears*)h; }
// n_mel, n_ch, n_embd, n_ff, n_head, n_head_kv, head_dim, window, n_out, d_conv, n_layer
void orc_ears_info(void* h, int* o) {
    auto* e = (ears*)h;
    const int v[11] = {e->n_mel, e->n_ch, e->n_embd, e->n_ff, e->n_head, e->n_head_kv, e->head_dim, e->window, e->n_out,
                       e->d_conv, (int)e->layers.size()};
    memcpy(o, v, sizeof(v));
}
// positions of a clip of n samples (ears.cpp:203-205)
int orc_ears_positions(void* h, int n) {
    auto* e = (ears*)h;
    const int n_pad = n <= e->n_fft ? e->n_fft : n + (e->hop - (n - e->n_fft) % e->hop) % e->hop;
    const int n_fr = (n_pad - e->n_fft) / e->hop + 1, T2 = (n_fr + 1) / 2, T4 = (T2 + 1) / 2;
    return (T4 + 1) / 2;
}
int orc_ears_frames(void* h, int n) {
    auto* e = (ears*)h;
    const int n_pad = n <= e->n_fft ? e->n_fft : n + (e->hop - (n - e->n_fft) % e->hop) % e->hop;
    return (n_pad - e->n_fft) / e->hop + 1;
}
// out [P][n_out]; mel (nullable) [n_frames][n_mel]; secs (nullable): wall seconds of the encode
int orc_ears_encode(void* h, const float* pcm, int n, float* out, float* mel, double* secs) {
    auto* e = (ears*)h;
    std::vector<float> o;
    const auto t0 = std::chrono::steady_clock::now();
    const int P = e->encode(pcm, n, o);
    if (secs) *secs = std::chrono::duration<double>(std::chrono::steady_clock::now() - t0).count();
    memcpy(out, o.data(), o.size() * sizeof(float));
    if (mel) memcpy(mel, e->last_mel.data(), e->last_mel.size() * sizeof(float));
    return P;
}
}
