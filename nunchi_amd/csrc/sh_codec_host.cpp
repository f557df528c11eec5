// Host side of the codec decoder on the device (imi/core/codec.{h,cpp}): load (Q8_0 tables repacked as the voice
// generator's), the per-frame launch sequence captured once as a HIP graph, the carried state (conv memory, key /
// value rings, overlap-add), and the C ABI.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstdlib>
#include <cstring>
#include <string>
#include <vector>

#include "../../include/seoul_hip.h"
#include "gguf_file.h"
#include "sh_codec.h"
#include "sh_voice.h"

namespace sh {
int set_error(int code, const std::string& msg);
}
using namespace sh;

namespace {
#define CCHK(x)                                                                                                 \
    do {                                                                                                        \
        hipError_t e_ = (x);                                                                                    \
        if (e_ != hipSuccess) return set_error(SH_E_HIP, std::string(#x) + ": " + hipGetErrorString(e_));       \
    } while (0)

struct clayer {
    bool conv = false;
    q8dev pw1, pw2, qkv, o, gate_up, down;
    const float *ln1 = nullptr, *ln2 = nullptr, *post1 = nullptr, *post2 = nullptr;
    const float *taps = nullptr, *gate_w = nullptr, *q_norm = nullptr, *k_norm = nullptr;
    float* mem = nullptr;                      // conv memory [d_conv][E]
    float *k_ring = nullptr, *v_ring = nullptr; // attention [CX_RING][kvd]
};
}  // namespace

struct sh_codec {
    int device = 0;
    hipStream_t stream = nullptr;
    sh_codec_shape info{};
    float eps = 1e-5f, theta = 1e6f;
    char* mem = nullptr;
    std::vector<clayer> layers;
    const float *lvl = nullptr, *qo_w = nullptr, *qo_b = nullptr, *in_b = nullptr, *out_b = nullptr, *out_norm = nullptr;
    q8dev* in_tab = nullptr;                   // device [1]: in_proj (the single-input kernel reads tables by index)
    q8dev out_proj;
    const float2* tw = nullptr;
    const float* hann = nullptr;
    float *ola = nullptr, *wsum = nullptr;
    float *v = nullptr, *x = nullptr, *big = nullptr, *u = nullptr, *act = nullptr, *y = nullptr, *spec = nullptr, *pcm = nullptr;
    float* frames = nullptr;   // [P][n_fft] the frame's inverse transforms before the overlap-add
    size_t state_bytes = 0;
    char* state = nullptr;                     // conv memory, rings, overlap: cleared by reset
    cframe_in* in_dev = nullptr;
    cframe_in* in_host = nullptr;              // pinned
    float* pcm_host = nullptr;                 // pinned [P][hop]
    int pos = 0, pad_left = 0;
    bool use_graph = true;
    hipGraphExec_t graph = nullptr;
};

namespace {

void release(sh_codec* c) {
    if (!c) return;
    (void)hipSetDevice(c->device);
    if (c->graph) (void)hipGraphExecDestroy(c->graph);
    if (c->stream) (void)hipStreamSynchronize(c->stream);
    if (c->mem) (void)hipFree(c->mem);
    if (c->in_host) (void)hipHostFree(c->in_host);
    if (c->pcm_host) (void)hipHostFree(c->pcm_host);
    if (c->stream) (void)hipStreamDestroy(c->stream);
    delete c;
}

int units_of(const q8dev& W) { return (W.rows_pad / 8 + 1) / 2; }   // the scaled order: two row groups per workgroup

int enqueue_frame(sh_codec* c) {
    const sh_codec_shape& I = c->info;
    const int E = I.n_embd, D = I.head_dim, nq = I.n_head * D, nr = (I.n_head + 2 * I.n_head_kv) * D;
    CCHK(launch_cfsq(cfsq_args{c->in_dev, c->lvl, c->qo_w, c->qo_b, I.n_lvl, I.n_q, c->v}, c->stream));
    vone_args va{};
    va.tabs = c->in_tab; va.rows = E; va.src = c->v; va.bias = c->in_b; va.head = 0; va.out = c->x; va.rows_per_wg = 64;
    CCHK(launch_vone(va, 1, I.n_q, c->stream));
    CCHK(launch_crep(crep_args{c->x, E}, c->stream));
    auto tab = [&](const q8dev& W, int pro, int epi, const float* src, int src_ld, const float* nw, float* out, int out_ld) {
        vtab_args t{};
        t.W = W; t.src = src; t.src_ld = src_ld; t.norm_w = nw; t.eps = c->eps; t.out = out; t.out_ld = out_ld;
        t.units = epi == VE_SWIGLU ? W.rows_pad / 16 : units_of(W);
        return launch_vtab(CX_P, pro, epi, t, c->stream);
    };
    for (const clayer& L : c->layers) {
        if (L.conv) {   // codec.cpp:163-192
            CCHK(tab(L.pw1, VP_NORM, VE_STORE, c->x, E, L.ln1, c->big, 3 * E));
            CCHK(launch_cconv(cconv_args{c->big, L.taps, L.mem, c->u, E, I.d_conv}, c->stream));
            CCHK(tab(L.pw2, VP_PLAIN, VE_STORE, c->u, E, nullptr, c->y, E));
        } else {        // codec.cpp:193-236
            CCHK(tab(L.qkv, VP_NORM, VE_STORE, c->x, E, L.ln1, c->big, nr));
            cattn_args aa{c->in_dev, c->big, nr, c->x, L.ln1, L.gate_w, L.q_norm, L.k_norm, L.k_ring, L.v_ring, c->act,
                          E, I.n_head, I.n_head_kv, D, c->eps};
            CCHK(launch_cattn(aa, c->stream));
            CCHK(tab(L.o, VP_PLAIN, VE_STORE, c->act, nq, nullptr, c->y, E));
        }
        CCHK(launch_cresid(cresid_args{c->y, L.post1, c->x, E, c->eps}, c->stream));
        CCHK(tab(L.gate_up, VP_NORM, VE_SWIGLU, c->x, E, L.ln2, c->act, I.n_ff));
        CCHK(tab(L.down, VP_PLAIN, VE_STORE, c->act, I.n_ff, nullptr, c->y, E));
        CCHK(launch_cresid(cresid_args{c->y, L.post2, c->x, E, c->eps}, c->stream));
    }
    CCHK(tab(c->out_proj, VP_NORM, VE_STORE, c->x, E, c->out_norm, c->spec, 2 * I.n_bins));
    CCHK(launch_cistft(cistft_args{c->spec, c->out_b, c->tw, c->hann, c->ola, c->wsum, c->pcm, c->frames}, c->stream));
    return SH_OK;
}

}  // namespace

extern "C" {

int sh_codec_load(int device, const char* path, sh_codec** out) {   // imi/core/codec.cpp:41-108
    if (!path || !out) return set_error(SH_E_ARG, "sh_codec_load: bad argument");
    *out = nullptr;
    CCHK(hipSetDevice(device));
    gg_file f;
    if (!f.load(path)) return set_error(SH_E_FILE, "sh_codec_load: " + f.error);
    const std::string g = "a.gen.wav.";
    const gg_tensor *cb = f.get(g + "quant.first.codebook.weight"), *qw = f.get(g + "quant.first.out_proj.weight");
    const gg_tensor *qb = f.get(g + "quant.first.out_proj.bias"), *ip = f.get(g + "tfm.in_proj.weight");
    const gg_tensor *ib = f.get(g + "tfm.in_proj.bias"), *op = f.get(g + "tfm.out_proj.weight"), *ob = f.get(g + "tfm.out_proj.bias");
    const gg_tensor* on = f.get(g + "tfm.output_norm.weight");
    if (!cb || !qw || !qb || !ip || !ib || !op || !ob || !on) return set_error(SH_E_FILE, "sh_codec_load: " + f.error);
    sh_codec_shape I{};
    I.n_lvl = (int)cb->ne[0];
    I.n_codes = (int)cb->ne[1];
    I.n_q = (int)ip->ne[0];
    I.n_embd = (int)ip->ne[1];
    I.n_bins = (int)op->ne[1] / 2;
    const int E = I.n_embd, nqin = CX_NCB * I.n_lvl;
    auto f32n = [&](const gg_tensor* t, int64_t n) { return t->type == GT_F32 && t->ne[0] * t->ne[1] * t->ne[2] * t->ne[3] == n; };
    if (cb->type != GT_F32 || I.n_lvl < 1 || I.n_lvl > 16 || I.n_codes < 1 || !f32n(qw, (int64_t)I.n_q * nqin) ||
        qw->ne[0] != nqin || !f32n(qb, I.n_q))
        return set_error(SH_E_SHAPE, "sh_codec_load: the quantizer's level table / projection are not as expected");
    if (ip->type != GT_Q8_0 || op->type != GT_Q8_0 || I.n_q % 32 || I.n_q > 4096 || E % 32 || E > 512 || op->ne[0] != E ||
        I.n_bins != CX_NB || !f32n(ib, E) || !f32n(ob, 2 * CX_NB) || !f32n(on, E))
        return set_error(SH_E_SHAPE, "sh_codec_load: in_proj / out_proj must be Q8_0, n_embd a multiple of 32 up to 512, "
                                     "641 bins");
    struct plan { std::vector<const uint8_t*> rows; int cols; q8dev* dst; };
    std::vector<plan> tabs;
    auto rows_of = [](std::vector<const uint8_t*>& o, const gg_tensor* t, int r0, int n) {
        for (int r = r0; r < r0 + n; r++) o.push_back(static_cast<const uint8_t*>(t->data) + (size_t)r * t->nb[1]);
    };
    std::vector<clayer> layers;
    for (int il = 0;; il++) {
        if (!f.get(g + "tfm.blk." + std::to_string(il) + ".ln1.weight", false)) break;
        layers.emplace_back();
    }
    if (layers.empty()) return set_error(SH_E_FILE, "sh_codec_load: no codec layers");
    struct vec { const gg_tensor* t; const float** dst; std::vector<float> host; };   // f32 vectors (host copy when converted)
    std::vector<vec> vecs;
    int n_conv = 0, n_attn = 0;
    for (size_t il = 0; il < layers.size(); il++) {
        const std::string p = g + "tfm.blk." + std::to_string(il) + ".";
        clayer& L = layers[il];
        const gg_tensor *l1 = f.get(p + "ln1.weight"), *l2 = f.get(p + "ln2.weight");
        const gg_tensor *p1 = f.get(p + "attn_post_norm.weight"), *p2 = f.get(p + "ffn_post_norm.weight");
        const gg_tensor *fg = f.get(p + "ffn_gate.weight"), *fu = f.get(p + "ffn_up.weight"), *fd = f.get(p + "ffn_down.weight");
        if (!l1 || !l2 || !p1 || !p2 || !fg || !fu || !fd) return set_error(SH_E_FILE, "sh_codec_load: " + f.error);
        if (!f32n(l1, E) || !f32n(l2, E) || !f32n(p1, E) || !f32n(p2, E))
            return set_error(SH_E_SHAPE, "sh_codec_load: layer norms must be f32 of n_embd");
        if (il == 0) I.n_ff = (int)fg->ne[1];
        if (fg->type != GT_Q8_0 || fu->type != GT_Q8_0 || fd->type != GT_Q8_0 || fg->ne[1] != I.n_ff || fu->ne[1] != I.n_ff ||
            fg->ne[0] != E || fu->ne[0] != E || fd->ne[1] != E || fd->ne[0] != I.n_ff || I.n_ff % 32 || I.n_ff > 4096)
            return set_error(SH_E_SHAPE, "sh_codec_load: FFN tables must be Q8_0, n_ff a multiple of 32 up to 4096");
        vecs.push_back({l1, &L.ln1, {}});
        vecs.push_back({l2, &L.ln2, {}});
        vecs.push_back({p1, &L.post1, {}});
        vecs.push_back({p2, &L.post2, {}});
        if (const gg_tensor* cw = f.get(p + "conv_dw.weight", false)) {
            const gg_tensor *w1 = f.get(p + "conv_pw1.weight"), *w2 = f.get(p + "conv_pw2.weight");
            if (!w1 || !w2) return set_error(SH_E_FILE, "sh_codec_load: " + f.error);
            const int K = (int)cw->ne[0];
            if (n_conv == 0) I.d_conv = K - 1;
            if (cw->type != GT_F32 || cw->ne[1] != E || K - 1 != I.d_conv || K < 2 || K > CX_MAX_TAPS ||
                w1->type != GT_Q8_0 || w2->type != GT_Q8_0 || w1->ne[1] != 3 * E || w1->ne[0] != E || w2->ne[1] != E || w2->ne[0] != E)
                return set_error(SH_E_SHAPE, "sh_codec_load: conv tables must be Q8_0 with 2 to 8 f32 taps");
            L.conv = true;
            vec tv{cw, &L.taps, std::vector<float>((size_t)K * E)};
            for (int e = 0; e < E; e++)   // [channel][tap] -> [tap][channel] (codec.cpp:65-67)
                for (int k = 0; k < K; k++) tv.host[(size_t)k * E + e] = static_cast<const float*>(cw->data)[(size_t)e * K + k];
            vecs.push_back(std::move(tv));
            plan a1{{}, E, &L.pw1}; rows_of(a1.rows, w1, 0, 3 * E); tabs.push_back(std::move(a1));
            plan a2{{}, E, &L.pw2}; rows_of(a2.rows, w2, 0, E); tabs.push_back(std::move(a2));
            n_conv++;
        } else {
            const gg_tensor *qn = f.get(p + "attn_q_norm.weight"), *kn = f.get(p + "attn_k_norm.weight");
            const gg_tensor *q = f.get(p + "attn_q.weight"), *k = f.get(p + "attn_k.weight"), *vv = f.get(p + "attn_v.weight");
            const gg_tensor *o = f.get(p + "attn_out.weight"), *gw = f.get(p + "attn_gate.weight");
            if (!qn || !kn || !q || !k || !vv || !o || !gw) return set_error(SH_E_FILE, "sh_codec_load: " + f.error);
            const int D = (int)qn->ne[0];
            if (n_attn == 0) {
                I.head_dim = D;
                I.n_head = (int)(q->ne[1] / D);
                I.n_head_kv = (int)(k->ne[1] / D);
            }
            if (D != I.head_dim || D % 32 || D > CX_MAX_D || I.n_head_kv < 1 || I.n_head % I.n_head_kv ||
                q->ne[1] != (int64_t)I.n_head * D || k->ne[1] != (int64_t)I.n_head_kv * D || vv->ne[1] != k->ne[1] ||
                q->ne[0] != E || k->ne[0] != E || vv->ne[0] != E || o->ne[1] != E || o->ne[0] != (int64_t)I.n_head * D ||
                gw->ne[0] != E || gw->ne[1] != I.n_head || (gw->type != GT_F32 && gw->type != GT_F16) || !f32n(qn, D) || !f32n(kn, D))
                return set_error(SH_E_SHAPE, "sh_codec_load: attention shapes not supported (head_dim a multiple of 32 up to 128)");
            for (const gg_tensor* t : {q, k, vv, o})
                if (t->type != GT_Q8_0) return set_error(SH_E_SHAPE, "sh_codec_load: attention tables must be Q8_0");
            vecs.push_back({qn, &L.q_norm, {}});
            vecs.push_back({kn, &L.k_norm, {}});
            vec gv{gw, &L.gate_w, std::vector<float>((size_t)I.n_head * E)};   // f16 gates widened (codec.cpp:86-87)
            for (size_t i = 0; i < gv.host.size(); i++)
                gv.host[i] = gw->type == GT_F16 ? [](uint16_t h) {
                    const uint32_t s = (h & 0x8000u) << 16, ex = (h >> 10) & 31, m = h & 1023;
                    uint32_t bits;
                    if (ex == 31) bits = s | 0x7F800000u | (m << 13);
                    else if (ex) bits = s | ((ex + 112) << 23) | (m << 13);
                    else if (m) { float fv = (float)m * 5.9604644775390625e-8f; memcpy(&bits, &fv, 4); bits |= s; }
                    else bits = s;
                    float r; memcpy(&r, &bits, 4); return r; }(static_cast<const uint16_t*>(gw->data)[i])
                                                  : static_cast<const float*>(gw->data)[i];
            vecs.push_back(std::move(gv));
            plan aq{{}, E, &L.qkv};   // q | k | v stacked (codec.cpp:80)
            for (const gg_tensor* t : {q, k, vv}) rows_of(aq.rows, t, 0, (int)t->ne[1]);
            tabs.push_back(std::move(aq));
            plan ao{{}, (int)o->ne[0], &L.o}; rows_of(ao.rows, o, 0, E); tabs.push_back(std::move(ao));
            n_attn++;
        }
        plan pg{{}, E, &L.gate_up};   // gate and up interleaved by 8-row group (codec.cpp:90-91)
        for (int t = 0; t < I.n_ff; t += 8) { rows_of(pg.rows, fg, t, 8); rows_of(pg.rows, fu, t, 8); }
        tabs.push_back(std::move(pg));
        plan pd{{}, I.n_ff, &L.down}; rows_of(pd.rows, fd, 0, E); tabs.push_back(std::move(pd));
    }
    if (n_attn == 0) { I.head_dim = 32; I.n_head = 1; I.n_head_kv = 1; }   // (unused: no attention layer)
    I.n_layer = (int)layers.size();
    auto* c = new sh_codec;
    c->device = device;
    q8dev in_tab_host{};
    {
        plan pi{{}, I.n_q, &in_tab_host}; rows_of(pi.rows, ip, 0, E); tabs.push_back(std::move(pi));
        plan po{{}, E, &c->out_proj}; rows_of(po.rows, op, 0, 2 * CX_NB); tabs.push_back(std::move(po));
    }
    vecs.push_back({cb, &c->lvl, {}});
    vecs.push_back({qw, &c->qo_w, {}});
    vecs.push_back({qb, &c->qo_b, {}});
    vecs.push_back({ib, &c->in_b, {}});
    vecs.push_back({ob, &c->out_b, {}});
    vecs.push_back({on, &c->out_norm, {}});
    c->layers = std::move(layers);
    c->use_graph = !(getenv("SEOUL_HIP_GRAPHS") && !strcmp(getenv("SEOUL_HIP_GRAPHS"), "0"));
    const int D = I.head_dim, kvd = I.n_head_kv * D, nq = I.n_head * D, nr = (I.n_head + 2 * I.n_head_kv) * D;

    size_t need = 0;
    auto room = [&](size_t n) { need += (n + 255) / 256 * 256; };
    for (const plan& t : tabs) {
        const size_t G = (t.rows.size() + 7) / 8, nb = t.cols / 32;
        room(G * nb * 256);
        room(G * nb * 16);
    }
    for (auto& vv : vecs) room((vv.host.empty() ? (size_t)(vv.t->ne[0] * vv.t->ne[1] * vv.t->ne[2] * vv.t->ne[3]) : vv.host.size()) * 4);
    room(sizeof(q8dev));
    room((size_t)CX_NFFT * sizeof(float2));
    room((size_t)CX_NFFT * 4);
    const size_t state0 = need;
    for (const clayer& L : c->layers) {
        if (L.conv) room((size_t)I.d_conv * E * 4);
        else { room((size_t)CX_RING * kvd * 4); room((size_t)CX_RING * kvd * 4); }
    }
    room((size_t)CX_NFFT * 4 * 2);
    const size_t state1 = need;
    room((size_t)I.n_q * 4);
    room((size_t)CX_P * E * 4);                                   // x
    room((size_t)CX_P * std::max(3 * E, nr) * 4);                 // big
    room((size_t)CX_P * E * 4);                                   // u
    room((size_t)CX_P * std::max(nq, I.n_ff) * 4);                // act
    room((size_t)CX_P * E * 4);                                   // y
    room((size_t)CX_P * 2 * CX_NB * 4);                           // spec
    room((size_t)CX_P * CX_HOP * 4);                              // pcm
    room((size_t)CX_P * CX_NFFT * 4);                             // frames
    room(sizeof(cframe_in));
    hipError_t e = hipStreamCreateWithFlags(&c->stream, hipStreamNonBlocking);
    if (e == hipSuccess) e = hipMalloc(&c->mem, need);
    if (e == hipSuccess) e = hipHostMalloc(reinterpret_cast<void**>(&c->in_host), sizeof(cframe_in), hipHostMallocDefault);
    if (e == hipSuccess) e = hipHostMalloc(reinterpret_cast<void**>(&c->pcm_host), (size_t)CX_P * CX_HOP * 4, hipHostMallocDefault);
    if (e != hipSuccess) {
        release(c);
        return set_error(SH_E_NOMEM, std::string("sh_codec_load: allocation: ") + hipGetErrorString(e));
    }
    size_t used = 0;
    auto take = [&](size_t n) { char* p = c->mem + used; used += (n + 255) / 256 * 256; return p; };
    std::vector<int8_t> codes;
    std::vector<uint16_t> scales;
    long long tb = 0;
    for (const plan& t : tabs) {
        repack_q8(t.rows, t.cols, codes, scales);
        q8dev d;
        d.rows = (int)t.rows.size();
        d.rows_pad = (d.rows + 7) / 8 * 8;
        d.cols = t.cols;
        d.nb = t.cols / 32;
        char* cp = take(codes.size());
        char* sp = take(scales.size() * 2);
        e = hipMemcpy(cp, codes.data(), codes.size(), hipMemcpyHostToDevice);
        if (e == hipSuccess) e = hipMemcpy(sp, scales.data(), scales.size() * 2, hipMemcpyHostToDevice);
        if (e != hipSuccess) { release(c); return set_error(SH_E_HIP, std::string("sh_codec_load: upload: ") + hipGetErrorString(e)); }
        d.codes = reinterpret_cast<const int8_t*>(cp);
        d.scales = reinterpret_cast<const uint16_t*>(sp);
        *t.dst = d;
        tb += (long long)d.rows * d.nb * 34;
    }
    for (auto& vv : vecs) {
        const size_t n = vv.host.empty() ? (size_t)(vv.t->ne[0] * vv.t->ne[1] * vv.t->ne[2] * vv.t->ne[3]) : vv.host.size();
        char* p = take(n * 4);
        e = hipMemcpy(p, vv.host.empty() ? vv.t->data : vv.host.data(), n * 4, hipMemcpyHostToDevice);
        if (e != hipSuccess) { release(c); return set_error(SH_E_HIP, std::string("sh_codec_load: upload: ") + hipGetErrorString(e)); }
        *vv.dst = reinterpret_cast<const float*>(p);
    }
    c->in_tab = reinterpret_cast<q8dev*>(take(sizeof(q8dev)));
    // twiddles and the periodic Hann window as imi makes them at load (codec.cpp:101-104), with the C library
    std::vector<float2> tw(CX_NFFT);
    std::vector<float> hann(CX_NFFT);
    for (int i = 0; i < CX_NFFT; i++) {
        hann[i] = 0.5f * (1.0f - cosf(2.0f * (float)M_PI * i / CX_NFFT));
        const float a = 2.0f * (float)M_PI * i / CX_NFFT;
        tw[i] = make_float2(cosf(a), sinf(a));
    }
    char* twp = take((size_t)CX_NFFT * sizeof(float2));
    char* hp = take((size_t)CX_NFFT * 4);
    e = hipMemcpy(c->in_tab, &in_tab_host, sizeof(q8dev), hipMemcpyHostToDevice);
    if (e == hipSuccess) e = hipMemcpy(twp, tw.data(), tw.size() * sizeof(float2), hipMemcpyHostToDevice);
    if (e == hipSuccess) e = hipMemcpy(hp, hann.data(), hann.size() * 4, hipMemcpyHostToDevice);
    if (e != hipSuccess) { release(c); return set_error(SH_E_HIP, std::string("sh_codec_load: upload: ") + hipGetErrorString(e)); }
    c->tw = reinterpret_cast<const float2*>(twp);
    c->hann = reinterpret_cast<const float*>(hp);
    if (used != state0) { release(c); return set_error(SH_E_NOMEM, "sh_codec_load: internal layout error"); }
    c->state = c->mem + used;
    for (clayer& L : c->layers) {
        if (L.conv) L.mem = reinterpret_cast<float*>(take((size_t)I.d_conv * E * 4));
        else {
            L.k_ring = reinterpret_cast<float*>(take((size_t)CX_RING * kvd * 4));
            L.v_ring = reinterpret_cast<float*>(take((size_t)CX_RING * kvd * 4));
        }
    }
    c->ola = reinterpret_cast<float*>(take((size_t)CX_NFFT * 4 * 2));
    c->wsum = c->ola + CX_NFFT;
    c->state_bytes = state1 - state0;
    c->v = reinterpret_cast<float*>(take((size_t)I.n_q * 4));
    c->x = reinterpret_cast<float*>(take((size_t)CX_P * E * 4));
    c->big = reinterpret_cast<float*>(take((size_t)CX_P * std::max(3 * E, nr) * 4));
    c->u = reinterpret_cast<float*>(take((size_t)CX_P * E * 4));
    c->act = reinterpret_cast<float*>(take((size_t)CX_P * std::max(nq, I.n_ff) * 4));
    c->y = reinterpret_cast<float*>(take((size_t)CX_P * E * 4));
    c->spec = reinterpret_cast<float*>(take((size_t)CX_P * 2 * CX_NB * 4));
    c->frames = reinterpret_cast<float*>(take((size_t)CX_P * CX_NFFT * 4));
    c->pcm = reinterpret_cast<float*>(take((size_t)CX_P * CX_HOP * 4));
    c->in_dev = reinterpret_cast<cframe_in*>(take(sizeof(cframe_in)));
    if (used > need) { release(c); return set_error(SH_E_NOMEM, "sh_codec_load: internal layout error"); }
    I.table_bytes = tb;
    c->info = I;
    const int rc = sh_codec_reset(c);
    if (rc != SH_OK) { release(c); return rc; }
    *out = c;
    return SH_OK;
}

int sh_codec_free(sh_codec* c) {
    release(c);
    return SH_OK;
}

int sh_codec_info(const sh_codec* c, sh_codec_shape* out) {
    if (!c || !out) return set_error(SH_E_ARG, "sh_codec_info: bad argument");
    *out = c->info;
    return SH_OK;
}

int sh_codec_reset(sh_codec* c) {   // codec.cpp:110-119
    if (!c) return set_error(SH_E_ARG, "sh_codec_reset: bad argument");
    CCHK(hipSetDevice(c->device));
    CCHK(hipMemsetAsync(c->state, 0, c->state_bytes, c->stream));
    CCHK(hipStreamSynchronize(c->stream));
    c->pos = 0;
    c->pad_left = (CX_NFFT - CX_HOP) / 2;
    return SH_OK;
}

int sh_codec_frame(sh_codec* c, const int32_t* codes, float* pcm, int* n_out) {   // codec.cpp:121-127
    if (!c || !codes || !pcm || !n_out) return set_error(SH_E_ARG, "sh_codec_frame: bad argument");
    for (int i = 0; i < CX_NCB; i++)
        if (codes[i] < 0 || codes[i] >= c->info.n_codes) return set_error(SH_E_ARG, "sh_codec_frame: code out of range");
    CCHK(hipSetDevice(c->device));
    cframe_in& in = *c->in_host;
    memcpy(in.codes, codes, sizeof in.codes);
    in.pos = c->pos;
    // rope of positions pos .. pos + 5 as imi's rope forms it (codec.cpp:11-19): th = position, times
    // theta^(-2/D) per pair, with the C library's powf / cosf / sinf
    const int D = c->info.head_dim;
    const float scale = powf(c->theta, -2.0f / (float)D);
    for (int p = 0; p < CX_P; p++) {
        float th = (float)(c->pos + p);
        for (int i = 0; i < D / 2; i++) {
            in.cs[p][i] = make_float2(cosf(th), sinf(th));
            th *= scale;
        }
    }
    CCHK(hipMemcpyAsync(c->in_dev, &in, sizeof in, hipMemcpyHostToDevice, c->stream));
    if (c->use_graph) {
        if (!c->graph) {
            hipGraph_t g = nullptr;
            CCHK(hipStreamBeginCapture(c->stream, hipStreamCaptureModeThreadLocal));
            const int rc = enqueue_frame(c);
            const hipError_t e = hipStreamEndCapture(c->stream, &g);
            if (rc != SH_OK || e != hipSuccess) {   // (the captured graph, if any, is not kept)
                if (g) (void)hipGraphDestroy(g);
                if (rc != SH_OK) return rc;
                return set_error(SH_E_HIP, std::string("sh_codec_frame: capture: ") + hipGetErrorString(e));
            }
            const hipError_t ei = hipGraphInstantiate(&c->graph, g, nullptr, nullptr, 0);
            (void)hipGraphDestroy(g);
            if (ei != hipSuccess) { c->graph = nullptr; return set_error(SH_E_HIP, std::string("sh_codec_frame: instantiate: ") + hipGetErrorString(ei)); }
        }
        CCHK(hipGraphLaunch(c->graph, c->stream));
    } else {
        const int rc = enqueue_frame(c);
        if (rc != SH_OK) return rc;
    }
    CCHK(hipMemcpyAsync(c->pcm_host, c->pcm, (size_t)CX_P * CX_HOP * 4, hipMemcpyDeviceToHost, c->stream));
    CCHK(hipStreamSynchronize(c->stream));
    c->pos += CX_P;
    const int drop = std::min(c->pad_left, CX_P * CX_HOP);   // the start padding (codec.cpp:264)
    c->pad_left -= drop;
    *n_out = CX_P * CX_HOP - drop;
    memcpy(pcm, c->pcm_host + drop, (size_t)*n_out * 4);
    return SH_OK;
}

int sh_codec_flush(sh_codec* c, float* pcm, int* n_out) {   // codec.cpp:271-277
    if (!c || !pcm || !n_out) return set_error(SH_E_ARG, "sh_codec_flush: bad argument");
    CCHK(hipSetDevice(c->device));
    std::vector<float> ow((size_t)2 * CX_NFFT);
    CCHK(hipMemcpyAsync(ow.data(), c->ola, ow.size() * 4, hipMemcpyDeviceToHost, c->stream));
    CCHK(hipStreamSynchronize(c->stream));
    const float *ola = ow.data(), *wsum = ow.data() + CX_NFFT;
    const int tail = CX_NFFT - CX_HOP, trim = (CX_NFFT - CX_HOP) / 2;
    for (int i = 0; i < tail - trim; i++) pcm[i] = wsum[i] > 1e-8f ? ola[i] / wsum[i] : ola[i];
    *n_out = tail - trim;
    return sh_codec_reset(c);
}

}  // extern "C"
