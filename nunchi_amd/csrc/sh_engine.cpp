// libseoul_hip: the brain step of imi's engine (imi/core/seoul.{h,cpp}) on one MI355X, behind the C ABI of
// include/seoul_hip.h. Host side: GGUF read, repack into the device layout, conversation states, and the step as
// a captured HIP graph of fused kernels (one per table read, with the norms, cuts and epilogues folded in, plus
// attention and the end of step; sh_kernels.hip).
#include "../../include/seoul_hip.h"

#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <memory>
#include <string>
#include <vector>

#include "gguf_file.h"
#include "sh_ctx.h"

using namespace sh;

namespace {
thread_local std::string g_err;
int fail(int code, const std::string& msg) {
    g_err = msg;
    return code;
}
#define HIPCHK(x)                                                                                          \
    do {                                                                                                   \
        hipError_t e_ = (x);                                                                               \
        if (e_ != hipSuccess) return fail(SH_E_HIP, std::string(#x) + ": " + hipGetErrorString(e_));       \
    } while (0)

// Q4_0 / Q4_1 rows (tensor, row) -> device layout in a host staging buffer: codes [rows][nb][16], scales and (Q4_1)
// block minima [rows/8][nb][8]. A table's rows are all Q4_0 or all Q4_1 (imi/core/tables.cpp:70-72).
// Replace a grow-on-demand device buffer: the new block is allocated before the old one is freed, so a failed
// allocation leaves the buffer (and the capacity the caller keeps for it) as they were.
hipError_t regrow(void** p, size_t bytes) {
    void* q = nullptr;
    const hipError_t e = hipMalloc(&q, bytes);
    if (e != hipSuccess) return e;
    if (*p) (void)hipFree(*p);
    *p = q;
    return hipSuccess;
}

// both staging buffers of the kernel-level API, or neither
hipError_t regrow2(float** x, float** y, size_t n_floats) {
    void* nx = nullptr;
    void* ny = nullptr;
    hipError_t e = hipMalloc(&nx, n_floats * 4);
    if (e == hipSuccess) e = hipMalloc(&ny, n_floats * 4);
    if (e != hipSuccess) {
        if (nx) (void)hipFree(nx);
        return e;
    }
    if (*x) (void)hipFree(*x);
    if (*y) (void)hipFree(*y);
    *x = static_cast<float*>(nx);
    *y = static_cast<float*>(ny);
    return hipSuccess;
}

bool repack_q4(const std::vector<std::pair<const gg_tensor*, int>>& rows, std::vector<uint8_t>& codes, std::vector<uint16_t>& scales,
               std::vector<uint16_t>& mins, int* cols) {
    if (rows.empty() || rows.size() % 8) return false;
    const gg_tensor* t0 = rows[0].first;
    if (t0->type != GT_Q4_0 && t0->type != GT_Q4_1) return false;
    for (auto& r : rows)
        if (!r.first->data || r.first->type != t0->type || r.first->ne[0] != t0->ne[0]) return false;
    const bool q41 = t0->type == GT_Q4_1;
    const size_t bb = q41 ? 20 : 18;   // block: fp16 d, (Q4_1: fp16 m,) 16 bytes of nibbles
    const int K = (int)t0->ne[0], nb = K / 32, R = (int)rows.size();
    codes.resize((size_t)R * nb * 16);
    scales.resize((size_t)R * nb);
    mins.assign(q41 ? (size_t)R * nb : 0, 0);
    for (int r = 0; r < R; r++) {
        const uint8_t* src = static_cast<const uint8_t*>(rows[r].first->data) + (size_t)rows[r].second * rows[r].first->nb[1];
        for (int j = 0; j < nb; j++) {
            const uint8_t* blk = src + (size_t)j * bb;
            const size_t so = ((size_t)(r / 8) * nb + j) * 8 + (r % 8);
            memcpy(&scales[so], blk, 2);
            if (q41) memcpy(&mins[so], blk + 2, 2);
            memcpy(&codes[((size_t)r * nb + j) * 16], blk + bb - 16, 16);
        }
    }
    *cols = K;
    return true;
}
// Q6_K rows -> the tiled device layout (q6dev): unit u = row * nbk + block; word w (16 bytes: 0-7 ql, 8-11 qh, 12 the
// scales) of unit u at [(u / 64) * 13 + w][u % 64]; d per unit. Units are padded to whole tiles with zeros.
void repack_q6k(const gg_tensor* t, std::vector<uint8_t>& codes, std::vector<uint16_t>& d) {
    const int nbk = (int)t->ne[0] / 256, rows = (int)t->ne[1];
    const size_t nunit = (size_t)rows * nbk, ntile = (nunit + 63) / 64;
    codes.assign(ntile * 13 * 64 * 16, 0);
    d.assign(ntile * 64, 0);
    for (size_t u = 0; u < nunit; u++) {
        const uint8_t* blk = static_cast<const uint8_t*>(t->data) + (u / nbk) * t->nb[1] + (u % nbk) * 210;
        uint8_t* base = &codes[(u / 64) * 13 * 64 * 16 + (u % 64) * 16];
        for (int w = 0; w < 13; w++) memcpy(base + (size_t)w * 64 * 16, blk + 16 * w, 16);   // ql | qh | scales
        memcpy(&d[u], blk + 208, 2);
    }
}
size_t q6k_device_bytes(const gg_tensor* t) {
    const size_t ntile = ((size_t)t->ne[1] * (t->ne[0] / 256) + 63) / 64;
    return (ntile * 13 * 64 * 16 + 255) / 256 * 256 + (ntile * 64 * 2 + 255) / 256 * 256;
}
}  // namespace

namespace sh {
int set_error(int code, const std::string& msg) { return fail(code, msg); }   // for the other host files
}

namespace {
template <class T> void forget(std::vector<T*>& v, T* p) {
    for (size_t i = 0; i < v.size(); i++)
        if (v[i] == p) { v[i] = v.back(); v.pop_back(); return; }
}
void release_state_memory(sh_state* s) {
    if (s->kc) (void)hipFree(s->kc);
    if (s->vc) (void)hipFree(s->vc);
    if (s->conv) (void)hipFree(s->conv);
    s->kc = s->vc = nullptr;
    s->conv = nullptr;
}
}  // namespace

namespace {

// the event pair around this launch when sh_bench_step_kernel times this kind of launch (else none)
void probe_events(sh_ctx* c, int kind, hipEvent_t* t0, hipEvent_t* t1) {
    *t0 = *t1 = nullptr;
    if (!c->probe_ev || c->probe_kind != kind || 2 * (size_t)(c->probe_used + 1) > c->probe_ev->size()) return;
    *t0 = (*c->probe_ev)[2 * c->probe_used];
    *t1 = (*c->probe_ev)[2 * c->probe_used + 1];
    c->probe_used++;
}

int enqueue_step(sh_ctx* c, int M, bool want_logits) {
    const sh_model_info& I = c->info;
    const int E = I.n_embd;
    int cur = 0;
    auto base_args = [&]() {
        gemv_args a{};
        a.P = c->P_dev;
        a.E = E;
        a.eps = c->eps;
        return a;
    };
    auto units_of = [](const q4dev& t, int ug) { return t.rows / (8 * ug); };
    auto grid_of = [](int units) { return units < 4096 ? units : 4096; };
    const layer_dev* prev = nullptr;
    for (size_t il = 0; il < c->layers.size(); il++) {
        const layer_dev& L = c->layers[il];
        // first table read of the layer: its input is norm(x) after the previous layer's FFN residual
        gemv_args a = base_args();
        int pro;
        if (!prev) {
            pro = PRO_EMBED_NORM;
            a.emb = c->vocab;
            a.emb6 = c->vocab6;
            a.embd = c->embd_stage;
            a.x_out = c->xbuf[cur];
        } else {
            pro = PRO_RESID_NORM;
            a.x_in = c->xbuf[cur];
            a.y_in = c->fo;
            a.w_post = prev->post_ffn_norm;
            a.x_out = c->xbuf[cur ^ 1];
            cur ^= 1;
        }
        a.w_pre = L.attn_norm;
        if (L.conv) {
            a.W = L.in_proj;
            a.units = units_of(L.in_proj, 3);
            a.out = c->u;
            a.out_ld = E;
            a.conv_w = L.conv_w;
            a.conv_layer = L.ci;
            a.d_conv = I.d_conv;
            HIPCHK(launch_gemv(M, pro, EPI_CONV, grid_of(a.units), a, c->stream));
            gemv_args b = base_args();
            b.W = L.out_proj;
            b.units = units_of(L.out_proj, 1);
            b.src = c->u;
            b.src_ld = E;
            b.out = c->y;
            b.out_ld = E;
            HIPCHK(launch_gemv(M, PRO_CUT, EPI_STORE, grid_of(b.units), b, c->stream));
        } else {
            a.W = L.qkvg;
            a.units = units_of(L.qkvg, 1);
            a.out = c->qkv;
            a.out_ld = c->nqkv;
            HIPCHK(launch_gemv(M, pro, EPI_STORE, grid_of(a.units), a, c->stream));
            attn_args t{};
            t.qkv = c->qkv;
            t.ld_qkv = c->nqkv;
            t.att = c->att;
            t.q_norm = L.q_norm;
            t.k_norm = L.k_norm;
            t.rope_cs = L.swa ? c->rope_cs_swa : c->rope_cs;
            t.layer_ai = L.ai;
            t.n_head = I.n_head;
            t.n_kv = I.n_head_kv;
            t.D = I.head_dim;
            t.n_ctx = I.n_ctx;
            t.n_swa = L.swa ? I.n_swa : 0;
            t.eps = c->eps;
            t.P = c->P_dev;
            HIPCHK(launch_attn(M, t, c->stream));
            gemv_args b = base_args();
            b.W = L.o;
            b.units = units_of(L.o, 1);
            b.src = c->att;
            b.src_ld = I.n_head * I.head_dim;
            b.out = c->y;
            b.out_ld = E;
            HIPCHK(launch_gemv(M, PRO_CUT, EPI_STORE, grid_of(b.units), b, c->stream));
        }
        // FFN: x += norm(y) * post_attn_norm; h = norm(x) * ffn_norm; gate|up with SwiGLU; down
        gemv_args f = base_args();
        f.x_in = c->xbuf[cur];
        f.y_in = c->y;
        f.w_post = L.post_attn_norm;
        f.x_out = c->xbuf[cur ^ 1];
        cur ^= 1;
        f.w_pre = L.ffn_norm;
        f.W = L.gate_up;
        f.units = units_of(L.gate_up, 2);
        f.out = c->act;
        f.out_ld = I.n_ff;
        gemv_args d = base_args();
        d.W = L.down;
        d.units = units_of(L.down, 1);
        d.src = c->act;
        d.src_ld = I.n_ff;
        d.out = c->fo;
        d.out_ld = E;
        int dpro = PRO_CUT;
        if (c->use_precut && swiglu_cut_takes(M, f, d)) {   // gate|up cuts the activation once for every down workgroup
            f.upw = 4;
            f.outq = c->act_q;
            f.outd = c->act_d;
            f.outs = c->act_s;
            d.src_q = c->act_q;
            d.src_d = c->act_d;
            d.src_s = c->act_s;
            dpro = PRO_PRECUT;
        }
        hipEvent_t p0, p1;
        probe_events(c, 0, &p0, &p1);
        HIPCHK(launch_gemv(M, PRO_RESID_NORM, EPI_SWIGLU, grid_of(f.units), f, c->stream, p0, p1));
        probe_events(c, 1, &p0, &p1);
        HIPCHK(launch_gemv(M, dpro, EPI_STORE, grid_of(d.units), d, c->stream, p0, p1));
        prev = &L;
    }
    final_args z{};
    z.E = E;
    z.eps = c->eps;
    z.P = c->P_dev;
    z.advance = 1;
    if (want_logits) {
        gemv_args v = base_args();
        v.x_in = c->xbuf[cur];
        v.y_in = c->fo;
        v.w_post = prev->post_ffn_norm;
        v.w_pre = c->out_norm;
        v.hidden_out = c->hidden;
        v.W = c->vocab;
        v.W6 = c->vocab6;
        v.units = units_of(c->vocab, 1);
        v.out = c->logits;
        v.out_ld = I.n_vocab;
        v.part_v = c->part_v;
        v.part_i = c->part_i;
        const int grid = c->vocab6.codes ? SH_Q6K_GRID : gemv_logits_grid(M, PRO_RESID_NORM, v, c->vocab_grid);
        if (c->vocab6.codes) HIPCHK(launch_scores_q6k(M, grid, v, c->stream));
        else {
            hipEvent_t p0, p1;
            probe_events(c, 2, &p0, &p1);
            HIPCHK(launch_gemv(M, PRO_RESID_NORM, EPI_LOGITS, grid, v, c->stream, p0, p1));
        }
        z.part_v = c->part_v;
        z.part_i = c->part_i;
        z.n_part = grid;
        z.logits = c->logits;
        z.ld_logits = I.n_vocab;
    } else {
        z.x_in = c->xbuf[cur];
        z.y_in = c->fo;
        z.w_post = prev->post_ffn_norm;
        z.w_out = c->out_norm;
        z.hidden_out = c->hidden;
    }
    HIPCHK(launch_final(M, z, c->stream));
    return SH_OK;
}

int get_graph(sh_ctx* c, int M, bool want_logits, hipGraphExec_t* out) {
    if (!c->use_graphs) {
        *out = nullptr;
        return SH_OK;
    }
    hipGraphExec_t& g = c->graph[M][want_logits ? 1 : 0];
    if (!g) {
        hipGraph_t graph = nullptr;
        HIPCHK(hipStreamBeginCapture(c->stream, hipStreamCaptureModeThreadLocal));
        const int rc = enqueue_step(c, M, want_logits);
        hipError_t e = hipStreamEndCapture(c->stream, &graph);
        if (rc != SH_OK || e != hipSuccess) {   // (the captured graph, if any, is not kept)
            if (graph) (void)hipGraphDestroy(graph);
            if (rc != SH_OK) return rc;
            return fail(SH_E_HIP, std::string("graph capture: ") + hipGetErrorString(e));
        }
        e = hipGraphInstantiate(&g, graph, nullptr, nullptr, 0);
        (void)hipGraphDestroy(graph);
        if (e != hipSuccess) { g = nullptr; return fail(SH_E_HIP, std::string("graph instantiate: ") + hipGetErrorString(e)); }
    }
    *out = g;
    return SH_OK;
}

void fill_state(step_params& p, int m, const sh_state* s) {
    p.pos[m] = s->pos;
    p.kc[m] = s->kc;
    p.vc[m] = s->vc;
    p.conv[m] = s->conv;
    p.out_tok[m] = nullptr;
}

// host-precomputed rotation table: for every position, cos/sin of th_i / ff[i] with th_0 = pos and
// th_{i+1} = th_i * base^(-2/D) in fp32 (imi/core/seoul.cpp:19-28), so the device uses the same angles
std::vector<float2> rope_table(int n_ctx, int D, float base, const float* ff) {
    std::vector<float2> t((size_t)n_ctx * (D / 2));
    const float scale = powf(base, -2.0f / (float)D);
    for (int p = 0; p < n_ctx; p++) {
        float th = (float)p;
        for (int i = 0; i < D / 2; i++) {
            const float ang = th / (ff ? ff[i] : 1.0f);
            t[(size_t)p * (D / 2) + i] = make_float2(cosf(ang), sinf(ang));
            th *= scale;
        }
    }
    return t;
}


// The keys and tensor shapes of a brain file (imi/core/seoul.cpp:93-142 reads the same keys and tensors), checked
// against what the kernels take before anything is uploaded: every table's type, rows and columns, the same kv head
// count and FFN width in every layer, and a context the attention kernels can hold (their score rows live in LDS).
// Fills I (n_ctx included) and the float keys. Host only.
struct model_keys {
    float eps = 1e-5f, rope_base = 1e6f, rope_base_swa = 1e4f;
};

int check_model(gg_file& f, int n_ctx, sh_model_info& I, model_keys& K) {
    const gg_tensor* te = f.get("token_embd.weight");
    if (!te) return fail(SH_E_FILE, "sh_load: " + f.error);
    if (te->type != GT_Q4_0 && te->type != GT_Q6_K) return fail(SH_E_SHAPE, "sh_load: word table must be Q6_K or Q4_0");
    I = sh_model_info{};
    I.n_embd = (int)te->ne[0];
    I.n_vocab = (int)te->ne[1];
    const int E = I.n_embd;
    if (E < 32 || E % 32 || E / 32 > 64) return fail(SH_E_SHAPE, "sh_load: n_embd must be a multiple of 32 and at most 2048");
    if (I.n_vocab < 1) return fail(SH_E_SHAPE, "sh_load: empty word table");
    if (te->type == GT_Q6_K && E != 256 && E != 512 && E != 1024 && E != 2048)
        return fail(SH_E_SHAPE, "sh_load: a Q6_K word table needs n_embd 256, 512, 1024 or 2048");
    K.eps = f.key_f("lfm3.attention.layer_norm_rms_epsilon", 1e-5f);
    K.rope_base = f.key_f("lfm3.rope.freq_base", 1e6f);
    K.rope_base_swa = f.key_f("lfm3.rope.freq_base_swa", 1e4f);
    I.n_swa = (int)f.key_i("lfm3.attention.sliding_window", 0);
    I.d_conv = (int)f.key_i("lfm3.shortconv.l_cache", 7) - 1;
    I.n_head = (int)f.key_i("lfm3.attention.head_count", 16);
    I.head_dim = (int)f.key_i("lfm3.attention.key_length", 128);
    I.n_layer = (int)f.key_i("lfm3.block_count", 0);
    I.n_ctx = n_ctx;
    if (I.n_layer < 1) return fail(SH_E_FILE, "sh_load: no layers");
    if (I.n_swa < 0) return fail(SH_E_SHAPE, "sh_load: negative sliding window");
    auto table = [&](const gg_tensor* t, int64_t rows, int64_t cols, const std::string& what) -> int {
        if (t->type != GT_Q4_0 && t->type != GT_Q4_1) return fail(SH_E_SHAPE, "sh_load: " + what + " must be Q4_0 or Q4_1");
        if (t->ne[1] != rows || t->ne[0] != cols || t->ne[2] != 1 || t->ne[3] != 1)
            return fail(SH_E_SHAPE, "sh_load: " + what + " is " + std::to_string(t->ne[1]) + " x " + std::to_string(t->ne[0]) +
                                        ", the kernels need " + std::to_string(rows) + " x " + std::to_string(cols));
        return SH_OK;
    };
    int n_kv = -1, n_ff = -1, n_attn = 0;
    const int D = I.head_dim, Hq = I.n_head * D;
    for (int il = 0; il < I.n_layer; il++) {
        const std::string p = "blk." + std::to_string(il) + ".";
        int rc = SH_OK;
        if (const gg_tensor* cw = f.get(p + "shortconv.conv.weight", false)) {
            if (I.d_conv < 1 || I.d_conv > 8) return fail(SH_E_SHAPE, "sh_load: conv kernel must be 2 to 9 taps");
            if (cw->type != GT_F32 || cw->ne[1] != E || cw->ne[0] != I.d_conv + 1) return fail(SH_E_SHAPE, "sh_load: conv weight shape");
            const gg_tensor* ip = f.get(p + "shortconv.in_proj.weight");
            const gg_tensor* op = f.get(p + "shortconv.out_proj.weight");
            if (!ip || !op) return fail(SH_E_FILE, "sh_load: " + f.error);
            if ((rc = table(ip, 3LL * E, E, p + "shortconv.in_proj")) != SH_OK) return rc;
            if ((rc = table(op, E, E, p + "shortconv.out_proj")) != SH_OK) return rc;
        } else {
            const gg_tensor *q = f.get(p + "attn_q.weight"), *k = f.get(p + "attn_k.weight"), *v = f.get(p + "attn_v.weight");
            const gg_tensor *g = f.get(p + "attn_gate.weight"), *o = f.get(p + "attn_output.weight");
            if (!q || !k || !v || !g || !o) return fail(SH_E_FILE, "sh_load: " + f.error);
            if (D != 32 && D != 64 && D != 128) return fail(SH_E_SHAPE, "sh_load: head_dim must be 32, 64 or 128");
            if (I.n_head < 1 || Hq / 32 > 64) return fail(SH_E_SHAPE, "sh_load: attention width must be 32 to 2048");
            const int kv = k->ne[1] % D == 0 ? (int)(k->ne[1] / D) : 0;
            if (kv < 1 || I.n_head % kv || I.n_head / kv > 8)
                return fail(SH_E_SHAPE, "sh_load: " + p + "attn_k rows must be a multiple of head_dim giving 1 to 8 query heads per kv head");
            if (n_kv >= 0 && kv != n_kv) return fail(SH_E_SHAPE, "sh_load: kv head count differs between layers");
            n_kv = kv;
            if ((rc = table(q, Hq, E, p + "attn_q")) != SH_OK || (rc = table(k, (int64_t)kv * D, E, p + "attn_k")) != SH_OK ||
                (rc = table(v, (int64_t)kv * D, E, p + "attn_v")) != SH_OK || (rc = table(g, I.n_head, E, p + "attn_gate")) != SH_OK ||
                (rc = table(o, E, Hq, p + "attn_output")) != SH_OK)
                return rc;
            for (const char* nm : {"attn_q_norm.weight", "attn_k_norm.weight"}) {
                const gg_tensor* t = f.get(p + nm);
                if (!t) return fail(SH_E_FILE, "sh_load: " + f.error);
                if (t->type != GT_F32 || t->ne[0] * t->ne[1] != D) return fail(SH_E_SHAPE, "sh_load: " + p + nm + " must be f32 [head_dim]");
            }
            n_attn++;
        }
        for (const char* nm : {"attn_norm.weight", "post_attention_norm.weight", "ffn_norm.weight", "post_ffw_norm.weight"}) {
            const gg_tensor* t = f.get(p + nm);
            if (!t) return fail(SH_E_FILE, "sh_load: " + f.error);
            if (t->type != GT_F32 || t->ne[0] * t->ne[1] != E) return fail(SH_E_SHAPE, "sh_load: " + p + nm + " must be f32 [n_embd]");
        }
        const gg_tensor *fg = f.get(p + "ffn_gate.weight"), *fu = f.get(p + "ffn_up.weight"), *fd = f.get(p + "ffn_down.weight");
        if (!fg || !fu || !fd) return fail(SH_E_FILE, "sh_load: " + f.error);
        const int ff = (int)fg->ne[1];
        if (ff < 32 || ff % 32 || ff / 32 > 256) return fail(SH_E_SHAPE, "sh_load: n_ff must be a multiple of 32, at most 8192");
        if (n_ff >= 0 && ff != n_ff) return fail(SH_E_SHAPE, "sh_load: FFN width differs between layers");
        n_ff = ff;
        if ((rc = table(fg, ff, E, p + "ffn_gate")) != SH_OK || (rc = table(fu, ff, E, p + "ffn_up")) != SH_OK ||
            (rc = table(fd, E, ff, p + "ffn_down")) != SH_OK)
            return rc;
    }
    const gg_tensor* on = f.get("output_norm.weight");
    if (!on || on->type != GT_F32 || on->ne[0] * on->ne[1] != E) return fail(SH_E_FILE, "sh_load: output_norm.weight missing or not f32 [n_embd]");
    if (const gg_tensor* rf = f.get("rope_freqs.weight", false))
        if (rf->type != GT_F32 || rf->ne[0] != D / 2) return fail(SH_E_SHAPE, "sh_load: rope_freqs shape");
    I.n_attn = n_attn;
    I.n_head_kv = n_kv > 0 ? n_kv : 0;
    I.n_ff = n_ff;
    if (n_attn > 0) {
        const int grp = I.n_head / I.n_head_kv, lim = std::min(attn_max_ctx(grp, D), pf_attn_max_ctx(grp, D));
        if (n_ctx > lim)
            return fail(SH_E_SHAPE, "sh_load: n_ctx " + std::to_string(n_ctx) + " is above the " + std::to_string(lim) +
                                        " positions the attention kernels hold at this head shape");
    }
    return SH_OK;
}

}  // namespace

extern "C" {

const char* sh_last_error(void) { return g_err.c_str(); }

int sh_create(int device, sh_ctx** out) {
    if (!out) return fail(SH_E_ARG, "sh_create: out is null");
    int n = 0;
    HIPCHK(hipGetDeviceCount(&n));
    if (device < 0 || device >= n) return fail(SH_E_ARG, "sh_create: no such device");
    HIPCHK(hipSetDevice(device));
    const int rs = noalloc_setup(device);   // the no-allocation entry point's scratch address on this device
    if (rs != SH_OK) return rs;
    auto c = std::make_unique<sh_ctx>();
    c->device = device;
    HIPCHK(hipStreamCreateWithFlags(&c->stream, hipStreamNonBlocking));
    HIPCHK(hipEventCreate(&c->ev0));
    HIPCHK(hipEventCreate(&c->ev1));
    HIPCHK(hipHostMalloc((void**)&c->P_host, sizeof(step_params), hipHostMallocDefault));
    HIPCHK(hipMalloc((void**)&c->P_dev, sizeof(step_params)));
    memset(c->P_host, 0, sizeof(step_params));
    const char* g = getenv("SEOUL_HIP_GRAPHS");
    c->use_graphs = !(g && g[0] == '0');
    const char* pf = getenv("SEOUL_HIP_PREFILL");
    c->use_prefill = !(pf && strcmp(pf, "0") == 0);
    const char* pc = getenv("SEOUL_HIP_PRECUT");
    c->use_precut = !(pc && strcmp(pc, "0") == 0);
    *out = c.release();
    return SH_OK;
}

int sh_destroy(sh_ctx* c) {
    if (!c) return SH_OK;
    (void)hipSetDevice(c->device);
    if (c->stream) (void)hipStreamSynchronize(c->stream);
    for (sh_state* s : c->states) { release_state_memory(s); s->ctx = nullptr; }   // handles stay valid, detached
    for (sh_q4* t : c->tables) { if (t->mem) (void)hipFree(t->mem); t->mem = nullptr; t->ctx = nullptr; }
    for (auto& row : c->graph)
        for (auto& g : row)
            if (g) (void)hipGraphExecDestroy(g);
    if (c->w.base) (void)hipFree(c->w.base);
    if (c->work.base) (void)hipFree(c->work.base);
    if (c->pf_mem) (void)hipFree(c->pf_mem);
    if (c->bench_x) (void)hipFree(c->bench_x);
    if (c->bench_y) (void)hipFree(c->bench_y);
    if (c->P_dev) (void)hipFree(c->P_dev);
    if (c->P_host) (void)hipHostFree(c->P_host);
    if (c->gen_out) (void)hipFree(c->gen_out);
    if (c->ev0) (void)hipEventDestroy(c->ev0);
    if (c->ev1) (void)hipEventDestroy(c->ev1);
    if (c->stream) (void)hipStreamDestroy(c->stream);
    delete c;
    return SH_OK;
}

int sh_check_model(const char* path, int n_ctx, sh_model_info* out) {
    if (!path || n_ctx < 1) return fail(SH_E_ARG, "sh_check_model: bad argument");
    gg_file f;
    if (!f.load(path)) return fail(SH_E_FILE, "sh_load: " + f.error);
    sh_model_info I;
    model_keys K;
    const int rc = check_model(f, n_ctx, I, K);
    if (rc == SH_OK && out) *out = I;
    return rc;
}

// imi/core/seoul.cpp:93-186; the tied word table is Q6_K (imi's format) or Q4_0; tables repacked into the device layout
int sh_load(sh_ctx* c, const char* path, int n_ctx) {
    if (!c || !path || n_ctx < 1) return fail(SH_E_ARG, "sh_load: bad argument");
    if (c->loaded) return fail(SH_E_STATE, "sh_load: a model is already loaded in this context");
    HIPCHK(hipSetDevice(c->device));
    gg_file f;
    if (!f.load(path)) return fail(SH_E_FILE, "sh_load: " + f.error);
    sh_model_info& I = c->info;
    model_keys K;
    const int rc = check_model(f, n_ctx, I, K);
    if (rc != SH_OK) return rc;
    const gg_tensor* te = f.get("token_embd.weight");
    const bool q6 = te->type == GT_Q6_K;
    c->eps = K.eps;
    c->rope_base = K.rope_base;
    c->rope_base_swa = K.rope_base_swa;
    const std::vector<int64_t> swa_pat = f.key_arr("lfm3.attention.sliding_window_pattern");
    const int E = I.n_embd;

    // first pass: shapes, and the bytes the device arena needs
    struct plan { std::vector<std::pair<const gg_tensor*, int>> rows; q4dev* dst; };
    std::vector<plan> tables;
    c->layers.assign(I.n_layer, layer_dev{});
    auto all_rows = [](std::vector<std::pair<const gg_tensor*, int>>& o, const gg_tensor* t, int r0, int n) {
        for (int r = r0; r < r0 + n; r++) o.push_back({t, r});
    };
    std::vector<std::pair<const float**, const gg_tensor*>> vecs;   // fp32 vectors to upload
    std::vector<std::vector<float>> conv_t;                          // conv weights transposed to [tap][channel]
    std::vector<const float**> conv_dst;
    int n_attn = 0, n_conv = 0;
    for (int il = 0; il < I.n_layer; il++) {
        const std::string p = "blk." + std::to_string(il) + ".";
        layer_dev& L = c->layers[il];
        auto need_f32 = [&](const std::string& name, const float** dst, int64_t n) -> bool {
            const gg_tensor* t = f.get(p + name);
            if (!t) return false;
            if (t->type != GT_F32 || t->ne[0] * t->ne[1] != n) { f.error = p + name + " must be f32"; return false; }
            vecs.push_back({dst, t});
            return true;
        };
        if (!need_f32("attn_norm.weight", &L.attn_norm, E) || !need_f32("post_attention_norm.weight", &L.post_attn_norm, E) ||
            !need_f32("ffn_norm.weight", &L.ffn_norm, E) || !need_f32("post_ffw_norm.weight", &L.post_ffn_norm, E))
            return fail(SH_E_FILE, "sh_load: " + f.error);
        if (const gg_tensor* cw = f.get(p + "shortconv.conv.weight", false)) {
            L.conv = true;
            L.ci = n_conv++;
            const int K = (int)cw->ne[0], C = (int)cw->ne[1];
            if (cw->type != GT_F32 || C != E || K != I.d_conv + 1) return fail(SH_E_SHAPE, "sh_load: conv weight shape");
            std::vector<float> tw((size_t)K * C);
            const float* src = static_cast<const float*>(cw->data);
            for (int e = 0; e < C; e++)
                for (int k = 0; k < K; k++) tw[(size_t)k * C + e] = src[(size_t)e * K + k];   // [channel][tap] -> [tap][channel]
            conv_t.push_back(std::move(tw));
            conv_dst.push_back(&L.conv_w);
            const gg_tensor* ip = f.get(p + "shortconv.in_proj.weight");
            const gg_tensor* op = f.get(p + "shortconv.out_proj.weight");
            if (!ip || !op) return fail(SH_E_FILE, "sh_load: " + f.error);
            if (ip->ne[1] != 3 * E) return fail(SH_E_SHAPE, "sh_load: in_proj must have 3 * n_embd rows");
            // b, c, x rows of 8 channels side by side, so one unit holds everything the conv of 8 channels needs
            plan pi;
            for (int t = 0; t < E; t += 8) { all_rows(pi.rows, ip, t, 8); all_rows(pi.rows, ip, E + t, 8); all_rows(pi.rows, ip, 2 * E + t, 8); }
            pi.dst = &L.in_proj;
            tables.push_back(std::move(pi));
            plan po;
            all_rows(po.rows, op, 0, (int)op->ne[1]);
            po.dst = &L.out_proj;
            tables.push_back(std::move(po));
        } else {
            const gg_tensor *q = f.get(p + "attn_q.weight"), *k = f.get(p + "attn_k.weight"), *v = f.get(p + "attn_v.weight");
            const gg_tensor *g = f.get(p + "attn_gate.weight"), *o = f.get(p + "attn_output.weight");
            if (!q || !k || !v || !g || !o) return fail(SH_E_FILE, "sh_load: " + f.error);
            I.n_head_kv = (int)(k->ne[1] / I.head_dim);
            if (!need_f32("attn_q_norm.weight", &L.q_norm, I.head_dim) || !need_f32("attn_k_norm.weight", &L.k_norm, I.head_dim))
                return fail(SH_E_FILE, "sh_load: " + f.error);
            plan pq;   // q | k | v | gate stacked (imi/core/seoul.cpp:147)
            for (const gg_tensor* t : {q, k, v, g}) all_rows(pq.rows, t, 0, (int)t->ne[1]);
            pq.dst = &L.qkvg;
            tables.push_back(std::move(pq));
            plan po;
            all_rows(po.rows, o, 0, (int)o->ne[1]);
            po.dst = &L.o;
            tables.push_back(std::move(po));
            L.ai = n_attn++;
            L.swa = il < (int)swa_pat.size() && swa_pat[il] != 0;
        }
        const gg_tensor *fg = f.get(p + "ffn_gate.weight"), *fu = f.get(p + "ffn_up.weight"), *fd = f.get(p + "ffn_down.weight");
        if (!fg || !fu || !fd) return fail(SH_E_FILE, "sh_load: " + f.error);
        I.n_ff = (int)fg->ne[1];
        plan pg;   // gate and up interleaved by 8-row group (imi/core/seoul.cpp:155-160)
        for (int t = 0; t < I.n_ff; t += 8) { all_rows(pg.rows, fg, t, 8); all_rows(pg.rows, fu, t, 8); }
        pg.dst = &L.gate_up;
        tables.push_back(std::move(pg));
        plan pd;
        all_rows(pd.rows, fd, 0, (int)fd->ne[1]);
        pd.dst = &L.down;
        tables.push_back(std::move(pd));
    }
    if (!q6) {
        plan pv;
        all_rows(pv.rows, te, 0, I.n_vocab);
        pv.dst = &c->vocab;
        tables.push_back(std::move(pv));
    }
    const gg_tensor* on = f.get("output_norm.weight");
    if (!on || on->type != GT_F32) return fail(SH_E_FILE, "sh_load: output_norm.weight missing or not f32");
    vecs.push_back({&c->out_norm, on});
    const gg_tensor* rf = f.get("rope_freqs.weight", false);
    I.n_attn = n_attn;
    c->n_conv = n_conv;
    if (n_attn > 0 && ((I.head_dim != 32 && I.head_dim != 64 && I.head_dim != 128) || I.n_head % I.n_head_kv || I.n_head / I.n_head_kv > 8))
        return fail(SH_E_SHAPE, "sh_load: attention shape not supported (head_dim 32, 64 or 128, group <= 8)");
    if (n_attn > 0 && (I.n_head * I.head_dim) / 32 > 64) return fail(SH_E_SHAPE, "sh_load: attention width above 2048");
    if (I.n_ff % 32 || I.n_ff / 32 > 256) return fail(SH_E_SHAPE, "sh_load: n_ff must be a multiple of 32, at most 8192");
    c->nqkv = I.n_head * I.head_dim + 2 * I.n_head_kv * I.head_dim + I.n_head;
    if (c->nqkv % 8) return fail(SH_E_SHAPE, "sh_load: q|k|v|gate rows not a multiple of 8");

    // device arena: tables, fp32 vectors, conv weights, rope tables
    size_t need = 0;
    for (auto& t : tables) {
        const size_t nb = (size_t)t.rows[0].first->ne[0] / 32;
        need += (t.rows.size() * nb * 16 + 255) / 256 * 256 + 2 * ((t.rows.size() * nb * 2 + 255) / 256 * 256);   // + Q4_1 minima
    }
    if (q6) need += q6k_device_bytes(te);
    for (auto& v : vecs) need += ((size_t)v.second->nbytes + 255) / 256 * 256;
    for (auto& v : conv_t) need += (v.size() * 4 + 255) / 256 * 256;
    const size_t rope_bytes = ((size_t)n_ctx * (I.head_dim / 2) * sizeof(float2) + 255) / 256 * 256;
    need += 2 * rope_bytes + 4096;
    HIPCHK(hipMalloc((void**)&c->w.base, need));
    c->w.size = need;
    long long table_bytes = 0;
    std::vector<uint8_t> codes;
    std::vector<uint16_t> scales, mins;
    for (auto& t : tables) {
        int K = 0;
        if (!repack_q4(t.rows, codes, scales, mins, &K))
            return fail(SH_E_SHAPE, "sh_load: a table is not all Q4_0 or all Q4_1 with rows in multiples of 8");
        void* dc = c->w.take(codes.size());
        void* ds = c->w.take(scales.size() * 2);
        void* dm = mins.empty() ? nullptr : c->w.take(mins.size() * 2);
        if (!dc || !ds || (!mins.empty() && !dm)) return fail(SH_E_NOMEM, "sh_load: arena overflow");
        HIPCHK(hipMemcpy(dc, codes.data(), codes.size(), hipMemcpyHostToDevice));
        HIPCHK(hipMemcpy(ds, scales.data(), scales.size() * 2, hipMemcpyHostToDevice));
        if (dm) HIPCHK(hipMemcpy(dm, mins.data(), mins.size() * 2, hipMemcpyHostToDevice));
        t.dst->codes = dc;
        t.dst->scales = ds;
        t.dst->mins = dm;
        t.dst->rows = (int)t.rows.size();
        t.dst->cols = K;
        t.dst->nb = K / 32;
        table_bytes += (long long)(codes.size() + scales.size() * 2 + mins.size() * 2);
    }
    if (q6) {
        repack_q6k(te, codes, scales);
        void* dc = c->w.take(codes.size());
        void* dd = c->w.take(scales.size() * 2);
        if (!dc || !dd) return fail(SH_E_NOMEM, "sh_load: arena overflow");
        HIPCHK(hipMemcpy(dc, codes.data(), codes.size(), hipMemcpyHostToDevice));
        HIPCHK(hipMemcpy(dd, scales.data(), scales.size() * 2, hipMemcpyHostToDevice));
        c->vocab6.codes = dc;
        c->vocab6.d = static_cast<const uint16_t*>(dd);
        c->vocab6.rows = I.n_vocab;
        c->vocab6.cols = E;
        c->vocab6.nbk = E / 256;
        table_bytes += (long long)I.n_vocab * (E / 256) * 210;
    }
    for (auto& v : vecs) {
        void* d = c->w.take(v.second->nbytes);
        if (!d) return fail(SH_E_NOMEM, "sh_load: arena overflow");
        HIPCHK(hipMemcpy(d, v.second->data, v.second->nbytes, hipMemcpyHostToDevice));
        *v.first = static_cast<const float*>(d);
    }
    for (size_t i = 0; i < conv_t.size(); i++) {
        void* d = c->w.take(conv_t[i].size() * 4);
        if (!d) return fail(SH_E_NOMEM, "sh_load: arena overflow");
        HIPCHK(hipMemcpy(d, conv_t[i].data(), conv_t[i].size() * 4, hipMemcpyHostToDevice));
        *conv_dst[i] = static_cast<const float*>(d);
    }
    if (n_attn > 0) {
        const float* ff = rf ? static_cast<const float*>(rf->data) : nullptr;
        if (rf && (rf->type != GT_F32 || rf->ne[0] != I.head_dim / 2)) return fail(SH_E_SHAPE, "sh_load: rope_freqs shape");
        auto t = rope_table(n_ctx, I.head_dim, c->rope_base, ff);
        void* d = c->w.take(t.size() * sizeof(float2));
        HIPCHK(hipMemcpy(d, t.data(), t.size() * sizeof(float2), hipMemcpyHostToDevice));
        c->rope_cs = static_cast<const float2*>(d);
        auto t2 = rope_table(n_ctx, I.head_dim, c->rope_base_swa, nullptr);   // window layers: no freq factors
        void* d2 = c->w.take(t2.size() * sizeof(float2));
        HIPCHK(hipMemcpy(d2, t2.data(), t2.size() * sizeof(float2), hipMemcpyHostToDevice));
        c->rope_cs_swa = static_cast<const float2*>(d2);
    }
    I.table_bytes = table_bytes;
    {
        long long vb = 4LL * E;   // output norm
        for (const layer_dev& L : c->layers) {
            vb += 4LL * 4 * E;   // attn, post-attention, ffn, post-ffn norms
            if (L.conv) vb += 4LL * (I.d_conv + 1) * E + 2 * 4LL * I.d_conv * E;   // taps, memory read + written
            else vb += 4LL * 2 * I.head_dim;                                        // q and k norms
        }
        I.vector_bytes = vb;
    }
    f.drop_data();

    // work buffers for up to two conversations
    const int Hq = I.n_head * I.head_dim;
    const size_t fl = sizeof(float);
    const size_t work_need = fl * (2 * 2 * E + 2 * E + 2 * E + 2 * (size_t)c->nqkv + 2 * (size_t)Hq + 2 * (size_t)I.n_ff + 2 * E + 2 * E +
                                   2 * (size_t)I.n_vocab + 2 * E + 2 * (size_t)c->vocab_grid + 2 * 2 * (size_t)(I.n_ff / 32 + 1)) +
                             sizeof(int) * 2 * (size_t)c->vocab_grid + 2 * (size_t)I.n_ff + 32 * 256;
    HIPCHK(hipMalloc((void**)&c->work.base, work_need));
    c->work.size = work_need;
    HIPCHK(hipMemset(c->work.base, 0, work_need));
    auto fa = [&](size_t n) { return static_cast<float*>(c->work.take(n * fl)); };
    c->xbuf[0] = fa(2 * E);
    c->xbuf[1] = fa(2 * E);
    c->y = fa(2 * E);
    c->u = fa(2 * E);
    c->qkv = fa(2 * (size_t)c->nqkv);
    c->att = fa(2 * (size_t)Hq);
    c->act = fa(2 * (size_t)I.n_ff);
    c->fo = fa(2 * E);
    c->hidden = fa(2 * E);
    c->logits = fa(2 * (size_t)I.n_vocab);
    c->embd_stage = fa(2 * E);
    c->part_v = fa(2 * (size_t)c->vocab_grid);
    c->part_i = static_cast<int*>(c->work.take(sizeof(int) * 2 * (size_t)c->vocab_grid));
    c->act_q = static_cast<int8_t*>(c->work.take(2 * (size_t)I.n_ff));
    c->act_d = fa(2 * (size_t)(I.n_ff / 32 + 1));
    c->act_s = fa(2 * (size_t)(I.n_ff / 32 + 1));
    if (!c->part_i) return fail(SH_E_NOMEM, "sh_load: work arena overflow");
    HIPCHK(hipDeviceSynchronize());
    c->loaded = true;
    return SH_OK;
}

int sh_info(const sh_ctx* c, sh_model_info* out) {
    if (!c || !out) return fail(SH_E_ARG, "sh_info: null");
    if (!c->loaded) return fail(SH_E_STATE, "sh_info: no model loaded");
    *out = c->info;
    return SH_OK;
}

int sh_state_new(sh_ctx* c, sh_state** out) {
    if (!c || !out) return fail(SH_E_ARG, "sh_state_new: null");
    if (!c->loaded) return fail(SH_E_STATE, "sh_state_new: no model loaded");
    HIPCHK(hipSetDevice(c->device));
    const sh_model_info& I = c->info;
    auto s = std::make_unique<sh_state>();
    s->ctx = c;
    const size_t kv = (size_t)I.n_attn * I.n_head_kv * I.n_ctx * I.head_dim;
    const size_t cv = (size_t)c->n_conv * I.d_conv * I.n_embd;
    if (kv) {
        HIPCHK(hipMalloc((void**)&s->kc, kv * 2));
        HIPCHK(hipMalloc((void**)&s->vc, kv * 2));
        HIPCHK(hipMemset(s->kc, 0, kv * 2));
        HIPCHK(hipMemset(s->vc, 0, kv * 2));
    }
    if (cv) {
        HIPCHK(hipMalloc((void**)&s->conv, cv * 4));
        HIPCHK(hipMemset(s->conv, 0, cv * 4));
    }
    HIPCHK(hipDeviceSynchronize());
    c->states.push_back(s.get());
    *out = s.release();
    return SH_OK;
}

int sh_state_free(sh_state* s) {
    if (!s) return SH_OK;
    if (s->ctx) {   // a state whose context was destroyed has no device memory left
        (void)hipSetDevice(s->ctx->device);
        (void)hipStreamSynchronize(s->ctx->stream);
        release_state_memory(s);
        forget(s->ctx->states, s);
    }
    delete s;
    return SH_OK;
}

int sh_state_reset(sh_state* s) {
    if (!s) return fail(SH_E_ARG, "sh_state_reset: null");
    if (!s->ctx) return fail(SH_E_STATE, "sh_state_reset: its context was destroyed");
    sh_ctx* c = s->ctx;
    HIPCHK(hipSetDevice(c->device));
    s->pos = 0;
    const size_t cv = (size_t)c->n_conv * c->info.d_conv * c->info.n_embd;
    if (cv) HIPCHK(hipMemsetAsync(s->conv, 0, cv * 4, c->stream));
    HIPCHK(hipStreamSynchronize(c->stream));
    return SH_OK;
}

int sh_state_pos(const sh_state* s, int* pos) {
    if (!s || !pos) return fail(SH_E_ARG, "sh_state_pos: null");
    *pos = s->pos;
    return SH_OK;
}

int sh_state_set_pos(sh_state* s, int pos) {
    if (!s || !s->ctx) return fail(SH_E_STATE, "sh_state_set_pos: no state or its context was destroyed");
    if (pos < 0 || pos > s->ctx->info.n_ctx) return fail(SH_E_ARG, "sh_state_set_pos: out of range");
    s->pos = pos;
    return SH_OK;
}

static int run_step(sh_ctx* c, int M, sh_state* const st[2], const int32_t tok[2], const float* const emb[2], bool want_logits,
                    float* const hid[2], float* const lg[2], int32_t* const best[2]) {
    const sh_model_info& I = c->info;
    for (int m = 0; m < M; m++) {
        if (!st[m] || st[m]->ctx != c) return fail(SH_E_STATE, "step: state belongs to another context");
        if (tok[m] >= I.n_vocab) return fail(SH_E_ARG, "step: token id out of range");
        if (tok[m] < 0 && !emb[m]) return fail(SH_E_ARG, "step: token < 0 needs an input vector");
        if (st[m]->pos >= I.n_ctx) {
            fprintf(stderr, "seoul-hip: context full (%d)\n", I.n_ctx);
            return fail(SH_E_CONTEXT_FULL, "step: context full");
        }
    }
    if (M == 2 && st[0] == st[1]) return fail(SH_E_ARG, "step2: the two conversations must be different states");
    HIPCHK(hipSetDevice(c->device));
    hipGraphExec_t g;
    int rc = get_graph(c, M, want_logits, &g);
    if (rc != SH_OK) return rc;
    step_params& P = *c->P_host;
    memset(&P, 0, sizeof P);
    for (int m = 0; m < M; m++) {
        P.token[m] = tok[m];
        fill_state(P, m, st[m]);
        if (tok[m] < 0) HIPCHK(hipMemcpyAsync(c->embd_stage + (size_t)m * I.n_embd, emb[m], (size_t)I.n_embd * 4, hipMemcpyHostToDevice, c->stream));
    }
    HIPCHK(hipMemcpyAsync(c->P_dev, &P, sizeof P, hipMemcpyHostToDevice, c->stream));
    if (g) HIPCHK(hipGraphLaunch(g, c->stream));
    else if ((rc = enqueue_step(c, M, want_logits)) != SH_OK) return rc;
    for (int m = 0; m < M; m++) {
        if (hid[m]) HIPCHK(hipMemcpyAsync(hid[m], c->hidden + (size_t)m * I.n_embd, (size_t)I.n_embd * 4, hipMemcpyDeviceToHost, c->stream));
        if (want_logits && lg[m]) HIPCHK(hipMemcpyAsync(lg[m], c->logits + (size_t)m * I.n_vocab, (size_t)I.n_vocab * 4, hipMemcpyDeviceToHost, c->stream));
    }
    HIPCHK(hipMemcpyAsync(&P, c->P_dev, sizeof P, hipMemcpyDeviceToHost, c->stream));
    HIPCHK(hipStreamSynchronize(c->stream));
    for (int m = 0; m < M; m++) {
        if (best[m]) *best[m] = want_logits ? P.best[m] : -1;
        st[m]->pos++;
    }
    return SH_OK;
}


int sh_step(sh_ctx* c, sh_state* s, int32_t token, const float* embd, int want_logits, float* hidden, float* logits, int32_t* best) {
    if (!c || !c->loaded) return fail(SH_E_STATE, "sh_step: no model loaded");
    sh_state* st[2] = {s, nullptr};
    const int32_t tok[2] = {token, 0};
    const float* emb[2] = {embd, nullptr};
    float* hid[2] = {hidden, nullptr};
    float* lg[2] = {logits, nullptr};
    int32_t* bs[2] = {best, nullptr};
    return run_step(c, 1, st, tok, emb, want_logits != 0, hid, lg, bs);
}

int sh_step2(sh_ctx* c, sh_state* a, int32_t ta, const float* ea, int la, sh_state* b, int32_t tb, const float* eb, int lb,
             float* ha, float* lga, int32_t* besta, float* hb, float* lgb, int32_t* bestb) {
    if (!c || !c->loaded) return fail(SH_E_STATE, "sh_step2: no model loaded");
    sh_state* st[2] = {a, b};
    const int32_t tok[2] = {ta, tb};
    const float* emb[2] = {ea, eb};
    float* hid[2] = {ha, hb};
    float* lg[2] = {la ? lga : nullptr, lb ? lgb : nullptr};
    int32_t* bs[2] = {la ? besta : nullptr, lb ? bestb : nullptr};
    if (besta && !la) *besta = -1;
    if (bestb && !lb) *bestb = -1;
    return run_step(c, 2, st, tok, emb, (la || lb), hid, lg, bs);
}

// n positions as n steps through the same graph (every position's numbers equal its own step's); a prefill
// that reads each table once per 64 positions replaces this path for long inputs
int sh_step_batch(sh_ctx* c, sh_state* s, const int32_t* tokens, const float* embd, int n, int want_logits,
                  float* hidden_last, float* logits, float* hidden_all, int32_t* best) {
    if (!c || !c->loaded) return fail(SH_E_STATE, "sh_step_batch: no model loaded");
    if (!s || n < 0 || (!tokens && !embd)) return fail(SH_E_ARG, "sh_step_batch: bad argument");
    const int E = c->info.n_embd;
    if (s->ctx != c) return fail(SH_E_STATE, "sh_step_batch: state belongs to another context");
    if (c->use_prefill && n >= 2) return run_prefill(c, s, tokens, embd, n, want_logits != 0, hidden_last, logits, hidden_all, best);
    if (s->pos + n > c->info.n_ctx) {
        fprintf(stderr, "seoul-hip: context full (%d)\n", c->info.n_ctx);
        return fail(SH_E_CONTEXT_FULL, "sh_step_batch: context full");
    }
    for (int i = 0; i < n; i++) {
        const bool last = i == n - 1;
        const int rc = sh_step(c, s, tokens ? tokens[i] : -1, embd ? embd + (size_t)i * E : nullptr, last && want_logits,
                               hidden_all ? hidden_all + (size_t)i * E : (last ? hidden_last : nullptr), last ? logits : nullptr,
                               last ? best : nullptr);
        if (rc != SH_OK) return rc;
        if (last && hidden_all && hidden_last) memcpy(hidden_last, hidden_all + (size_t)i * E, (size_t)E * 4);
    }
    return SH_OK;
}

int sh_generate(sh_ctx* c, sh_state* a, sh_state* b, int32_t fa, int32_t fb, int n, int32_t* out_a, int32_t* out_b, double* seconds) {
    if (!c || !c->loaded) return fail(SH_E_STATE, "sh_generate: no model loaded");
    if (!a || n < 0 || (b && b == a)) return fail(SH_E_ARG, "sh_generate: bad argument");
    const int M = b ? 2 : 1;
    sh_state* st[2] = {a, b};
    const int32_t first[2] = {fa, fb};
    for (int m = 0; m < M; m++) {
        if (st[m]->ctx != c) return fail(SH_E_STATE, "sh_generate: state belongs to another context");
        if (first[m] < 0 || first[m] >= c->info.n_vocab) return fail(SH_E_ARG, "sh_generate: first token out of range");
        if (st[m]->pos + n > c->info.n_ctx) {
            fprintf(stderr, "seoul-hip: context full (%d)\n", c->info.n_ctx);
            return fail(SH_E_CONTEXT_FULL, "sh_generate: context full");
        }
    }
    HIPCHK(hipSetDevice(c->device));
    if (n > c->gen_cap) {
        HIPCHK(regrow((void**)&c->gen_out, sizeof(int32_t) * 2 * (size_t)n));
        c->gen_cap = n;
    }
    hipGraphExec_t g;
    int rc = get_graph(c, M, true, &g);
    if (rc != SH_OK) return rc;
    step_params& P = *c->P_host;
    memset(&P, 0, sizeof P);
    P.greedy = 1;
    for (int m = 0; m < M; m++) {
        P.token[m] = first[m];
        fill_state(P, m, st[m]);
        P.out_tok[m] = c->gen_out + (size_t)m * c->gen_cap;
    }
    HIPCHK(hipMemcpyAsync(c->P_dev, &P, sizeof P, hipMemcpyHostToDevice, c->stream));
    HIPCHK(hipEventRecord(c->ev0, c->stream));
    for (int i = 0; i < n; i++) {
        if (g) HIPCHK(hipGraphLaunch(g, c->stream));
        else if ((rc = enqueue_step(c, M, true)) != SH_OK) return rc;
    }
    HIPCHK(hipEventRecord(c->ev1, c->stream));
    if (out_a) HIPCHK(hipMemcpyAsync(out_a, c->gen_out, sizeof(int32_t) * n, hipMemcpyDeviceToHost, c->stream));
    if (out_b && b) HIPCHK(hipMemcpyAsync(out_b, c->gen_out + c->gen_cap, sizeof(int32_t) * n, hipMemcpyDeviceToHost, c->stream));
    HIPCHK(hipStreamSynchronize(c->stream));
    float ms = 0.0f;
    HIPCHK(hipEventElapsedTime(&ms, c->ev0, c->ev1));
    if (seconds) *seconds = ms * 1e-3;
    for (int m = 0; m < M; m++) st[m]->pos += n;
    return SH_OK;
}

namespace {
// timing of individual kernel launches: event pairs recorded around each kernel (hipExtLaunchKernelGGL)
struct launch_timer {
    std::vector<hipEvent_t> ev;
    int used = 0;
    ~launch_timer() { for (auto e : ev) (void)hipEventDestroy(e); }
    hipError_t reserve(int n) {
        while ((int)ev.size() < 2 * n) {
            hipEvent_t e;
            const hipError_t r = hipEventCreate(&e);
            if (r != hipSuccess) return r;
            ev.push_back(e);
        }
        used = 0;
        return hipSuccess;
    }
    hipEvent_t start() { return ev[2 * used]; }
    hipEvent_t stop() { return ev[2 * used + 1]; }
    void next() { used++; }
    hipError_t total_ms(double* ms) {
        double t = 0;
        for (int i = 0; i < used; i++) {
            float x;
            const hipError_t r = hipEventElapsedTime(&x, ev[2 * i], ev[2 * i + 1]);
            if (r != hipSuccess) return r;
            t += x;
        }
        *ms = t;
        return hipSuccess;
    }
};

int bench_inputs(sh_ctx* c) {
    const size_t K = (size_t)(c->info.n_ff > c->info.n_embd ? c->info.n_ff : c->info.n_embd);
    const size_t R = 4 * (size_t)c->info.n_ff + 3 * (size_t)c->info.n_embd + 64;
    const size_t need = 2 * (K > R ? K : R);
    if (c->bench_cap >= need) return SH_OK;
    HIPCHK(regrow2(&c->bench_x, &c->bench_y, need));
    c->bench_cap = need;
    std::vector<float> in(c->bench_cap);
    for (size_t i = 0; i < in.size(); i++) in[i] = 0.01f * (float)((i * 7) % 13) - 0.06f;   // seoul.cpp:668
    HIPCHK(hipMemcpy(c->bench_x, in.data(), in.size() * 4, hipMemcpyHostToDevice));
    return SH_OK;
}
}  // namespace

int sh_bench_tables(sh_ctx* c, int ncol, int reps, double* ms_per_pass, double* avg_launch_us, double* bytes_per_pass, int* launches) {
    if (!c || !c->loaded) return fail(SH_E_STATE, "sh_bench_tables: no model loaded");
    if (ncol < 1 || ncol > 2 || reps < 1) return fail(SH_E_ARG, "sh_bench_tables: ncol in {1, 2}, reps >= 1");
    HIPCHK(hipSetDevice(c->device));
    int rc = bench_inputs(c);
    if (rc != SH_OK) return rc;
    const int K = c->info.n_ff > c->info.n_embd ? c->info.n_ff : c->info.n_embd;
    const int R = 4 * c->info.n_ff + 3 * c->info.n_embd + 64;
    std::vector<const q4dev*> ws;
    for (auto& L : c->layers)
        for (const q4dev* t : {&L.in_proj, &L.out_proj, &L.qkvg, &L.o, &L.gate_up, &L.down})
            if (t->rows) ws.push_back(t);
    double bytes = 0;
    for (auto* t : ws) bytes += (double)t->rows * t->nb * 18;
    launch_timer lt;
    HIPCHK(lt.reserve((int)ws.size()));
    double best = 1e30, total_launch_ms = 0;
    for (int r = 0; r < reps + 1; r++) {
        lt.used = 0;
        HIPCHK(hipEventRecord(c->ev0, c->stream));
        for (auto* t : ws) {
            gemv_args a{};
            a.W = *t;
            a.units = t->rows / 8;
            a.src = c->bench_x;
            a.src_ld = K;
            a.out = c->bench_y;
            a.out_ld = R;
            HIPCHK(launch_gemv(ncol, PRO_CUT, EPI_STORE, a.units < 4096 ? a.units : 4096, a, c->stream, lt.start(), lt.stop()));
            lt.next();
        }
        HIPCHK(hipEventRecord(c->ev1, c->stream));
        HIPCHK(hipEventSynchronize(c->ev1));
        float ms;
        HIPCHK(hipEventElapsedTime(&ms, c->ev0, c->ev1));
        double kms;
        HIPCHK(lt.total_ms(&kms));
        if (r == 0) continue;   // warm-up pass
        best = ms < best ? ms : best;
        total_launch_ms += kms;
    }
    if (ms_per_pass) *ms_per_pass = best;
    if (avg_launch_us) *avg_launch_us = total_launch_ms * 1e3 / reps / ws.size();
    if (bytes_per_pass) *bytes_per_pass = bytes;
    if (launches) *launches = (int)ws.size();
    return SH_OK;
}

// The step's own kernel for one table kind, launched with a real layer's arguments, rotating over the layers so
// successive launches read different tables (more than the 256 MB MALL in total); each launch timed by itself.
// bytes one FFN launch moves for M conversations: the table once, the fp32 vectors it reads and writes, and, when
// gate|up cuts the activation for down (pre-cut), the int8 codes and per-32 (d, s) pairs gate|up writes and down
// reads in place of the activation's floats
static double ffn_launch_bytes(const sh_ctx* c, const layer_dev& L, int kind, int M, bool precut) {
    const double E = c->info.n_embd, F = c->info.n_ff, cut = M * (F + 8.0 * (F / 32));
    if (kind == 0) return (double)L.gate_up.rows * L.gate_up.nb * 18 + 4.0 * M * (2 * E + F) + (precut ? cut : 0.0);
    return (double)L.down.rows * L.down.nb * 18 + 4.0 * M * E + (precut ? cut : 4.0 * M * F);
}

// whether the step runs layer L's FFN with the pre-cut (as enqueue_step decides)
static bool ffn_precut(const sh_ctx* c, const layer_dev& L, int M) {
    if (!c->use_precut) return false;
    gemv_args f{}, d{};
    f.E = c->info.n_embd;
    f.x_in = c->xbuf[0];
    f.y_in = c->y;
    f.w_post = L.post_attn_norm;
    f.W = L.gate_up;
    f.units = L.gate_up.rows / 16;
    f.out_ld = c->info.n_ff;
    d.W = L.down;
    return swiglu_cut_takes(M, f, d);
}

int sh_bench_kernel(sh_ctx* c, int kind, int M, int reps, double* avg_us, double* bytes_per_launch) {
    if (!c || !c->loaded) return fail(SH_E_STATE, "sh_bench_kernel: no model loaded");
    if (M < 1 || M > 2 || reps < 1 || kind < 0 || kind > 2) return fail(SH_E_ARG, "sh_bench_kernel: bad argument");
    HIPCHK(hipSetDevice(c->device));
    const sh_model_info& I = c->info;
    const int E = I.n_embd;
    launch_timer lt;
    HIPCHK(lt.reserve(reps));
    double bytes = 0;
    for (int pass = 0; pass < 2; pass++) {   // pass 0 warms up (code, TLB), pass 1 is timed
        lt.used = 0;
        bytes = 0;
        for (int r = 0; r < reps; r++) {
            const layer_dev& L = c->layers[r % c->layers.size()];
            gemv_args a{};
            a.P = c->P_dev;
            a.E = E;
            a.eps = c->eps;
            int pro, epi, grid;
            if (kind == 0) {          // FFN gate|up with the post-norm residual, RMS norm, cut, SwiGLU epilogue
                a.x_in = c->xbuf[0];
                a.y_in = c->y;
                a.w_post = L.post_attn_norm;
                a.x_out = c->xbuf[1];
                a.w_pre = L.ffn_norm;
                a.W = L.gate_up;
                a.units = L.gate_up.rows / 16;
                a.out = c->act;
                a.out_ld = I.n_ff;
                pro = PRO_RESID_NORM; epi = EPI_SWIGLU;
                const bool pc = ffn_precut(c, L, M);
                if (pc) {   // as in the step: the activation cut for down in the epilogue
                    a.upw = 4;
                    a.outq = c->act_q;
                    a.outd = c->act_d;
                    a.outs = c->act_s;
                }
                bytes += ffn_launch_bytes(c, L, 0, M, pc);
            } else if (kind == 1) {   // FFN down: input cut in the prologue, or taken as gate|up cut it
                a.W = L.down;
                a.units = L.down.rows / 8;
                a.src = c->act;
                a.src_ld = I.n_ff;
                a.out = c->fo;
                a.out_ld = E;
                pro = PRO_CUT; epi = EPI_STORE;
                const bool pc = ffn_precut(c, L, M);
                if (pc) {
                    a.src_q = c->act_q;
                    a.src_d = c->act_d;
                    a.src_s = c->act_s;
                    pro = PRO_PRECUT;
                }
                bytes += ffn_launch_bytes(c, L, 1, M, pc);
            } else {                  // word scores over the tied table
                a.x_in = c->xbuf[0];
                a.y_in = c->fo;
                a.w_post = L.post_ffn_norm;
                a.w_pre = c->out_norm;
                a.hidden_out = c->hidden;
                a.W = c->vocab;
                a.W6 = c->vocab6;
                a.units = c->vocab.rows / 8;
                a.out = c->logits;
                a.out_ld = I.n_vocab;
                a.part_v = c->part_v;
                a.part_i = c->part_i;
                pro = PRO_RESID_NORM; epi = EPI_LOGITS;
                bytes += c->vocab6.codes ? (double)I.n_vocab * (E / 256) * 210 + 4.0 * M * (2 * E + I.n_vocab)
                                         : (double)c->vocab.rows * c->vocab.nb * 18 + 4.0 * M * (2 * E + I.n_vocab);
            }
            if (kind == 2 && c->vocab6.codes) {
                HIPCHK(launch_scores_q6k(M, SH_Q6K_GRID, a, c->stream, lt.start(), lt.stop()));
                lt.next();
                continue;
            }
            grid = epi == EPI_LOGITS ? gemv_logits_grid(M, pro, a, c->vocab_grid) : (a.units < 4096 ? a.units : 4096);
            HIPCHK(launch_gemv(M, pro, epi, grid, a, c->stream, lt.start(), lt.stop()));
            lt.next();
        }
        HIPCHK(hipStreamSynchronize(c->stream));
    }
    double ms;
    HIPCHK(lt.total_ms(&ms));
    if (avg_us) *avg_us = ms * 1e3 / reps;
    if (bytes_per_launch) *bytes_per_launch = bytes / reps;
    return SH_OK;
}

// ---- kernel-level tables ----
// One kind of the step's own GEMV launches timed inside whole steps (0 FFN gate|up, 1 FFN down, 2 Q4_0 word
// scores): two untimed, then `steps` timed single (M = 1) or two-conversation steps run without the graph on fresh
// states fed seeded token ids; each launch of that kind records the events of its own dispatch, and its input is
// what the step's previous kernel has just written. Averages over every timed launch of that kind.
int sh_bench_step_kernel(sh_ctx* c, int kind, int M, int steps, double* avg_us, double* bytes_per_launch, int* launches) {
    if (!c || !c->loaded) return fail(SH_E_STATE, "sh_bench_step_kernel: no model loaded");
    if (M < 1 || M > 2 || kind < 0 || kind > 2 || steps < 1 || steps + 2 > c->info.n_ctx)
        return fail(SH_E_ARG, "sh_bench_step_kernel: kind in 0..2, M in {1, 2}, 1 <= steps <= n_ctx - 2");
    if (kind == 2 && c->vocab6.codes) return fail(SH_E_ARG, "sh_bench_step_kernel: the word table is not Q4_0");
    HIPCHK(hipSetDevice(c->device));
    const sh_model_info& I = c->info;
    const int per = kind == 2 ? 1 : (int)c->layers.size();
    struct guard {
        sh_ctx* c;
        sh_state* st[2] = {nullptr, nullptr};
        std::vector<hipEvent_t> ev;
        ~guard() {
            c->probe_ev = nullptr;
            c->probe_kind = -1;
            for (auto e : ev) (void)hipEventDestroy(e);
            for (auto s : st)
                if (s) (void)sh_state_free(s);
        }
    } g{c};
    for (int m = 0; m < M; m++) {
        const int rc = sh_state_new(c, &g.st[m]);
        if (rc != SH_OK) return rc;
    }
    g.ev.reserve(2 * (size_t)per * steps);
    for (size_t i = 0; i < 2 * (size_t)per * steps; i++) {
        hipEvent_t e;
        HIPCHK(hipEventCreate(&e));
        g.ev.push_back(e);
    }
    for (int s = 0; s < steps + 2; s++) {
        if (s == 2) {   // the first two steps warm the code and the tables' TLB entries
            c->probe_ev = &g.ev;
            c->probe_kind = kind;
            c->probe_used = 0;
        }
        step_params& P = *c->P_host;
        memset(&P, 0, sizeof P);
        for (int m = 0; m < M; m++) {
            P.token[m] = (int32_t)((7919LL * (s + 1) + 104729LL * m) % I.n_vocab);
            fill_state(P, m, g.st[m]);
        }
        HIPCHK(hipMemcpyAsync(c->P_dev, &P, sizeof P, hipMemcpyHostToDevice, c->stream));
        const int rc = enqueue_step(c, M, kind == 2);
        if (rc != SH_OK) return rc;
        HIPCHK(hipStreamSynchronize(c->stream));
        for (int m = 0; m < M; m++) g.st[m]->pos++;
    }
    const int n = c->probe_used;
    double ms = 0;
    for (int i = 0; i < n; i++) {
        float x;
        HIPCHK(hipEventElapsedTime(&x, g.ev[2 * i], g.ev[2 * i + 1]));
        ms += x;
    }
    double bytes = 0;
    for (const layer_dev& L : c->layers)
        if (kind != 2) bytes += ffn_launch_bytes(c, L, kind, M, ffn_precut(c, L, M));
    if (kind == 2) bytes = (double)c->vocab.rows * c->vocab.nb * 18 + 4.0 * M * (2 * I.n_embd + I.n_vocab);
    else bytes /= (double)c->layers.size();
    if (avg_us) *avg_us = n ? ms * 1e3 / n : 0.0;
    if (bytes_per_launch) *bytes_per_launch = bytes;
    if (launches) *launches = n;
    return SH_OK;
}

int sh_q4_create(sh_ctx* c, const void* q4_0, int rows, int cols, sh_q4** out) {
    if (!c || !q4_0 || !out || rows <= 0 || rows % 8 || cols <= 0 || cols % 32) return fail(SH_E_ARG, "sh_q4_create: rows % 8 == 0, cols % 32 == 0");
    if (cols / 32 > 4 * 64) return fail(SH_E_SHAPE, "sh_q4_create: at most 8192 columns");
    HIPCHK(hipSetDevice(c->device));
    gg_tensor t;
    t.type = GT_Q4_0;
    t.ne[0] = cols;
    t.ne[1] = rows;
    t.nb[1] = (size_t)cols / 32 * 18;
    t.data = q4_0;
    std::vector<std::pair<const gg_tensor*, int>> rr;
    for (int r = 0; r < rows; r++) rr.push_back({&t, r});
    std::vector<uint8_t> codes;
    std::vector<uint16_t> scales, mins;
    int K;
    if (!repack_q4(rr, codes, scales, mins, &K)) return fail(SH_E_SHAPE, "sh_q4_create: repack failed");
    auto h = std::make_unique<sh_q4>();
    h->ctx = c;
    const size_t cb = (codes.size() + 255) / 256 * 256;
    HIPCHK(hipMalloc(&h->mem, cb + scales.size() * 2));
    HIPCHK(hipMemcpy(h->mem, codes.data(), codes.size(), hipMemcpyHostToDevice));
    HIPCHK(hipMemcpy(static_cast<char*>(h->mem) + cb, scales.data(), scales.size() * 2, hipMemcpyHostToDevice));
    h->t.codes = h->mem;
    h->t.scales = static_cast<char*>(h->mem) + cb;
    h->t.rows = rows;
    h->t.cols = cols;
    h->t.nb = cols / 32;
    c->tables.push_back(h.get());
    *out = h.release();
    return SH_OK;
}

int sh_q4_free(sh_q4* t) {
    if (!t) return SH_OK;
    if (t->ctx) {
        (void)hipSetDevice(t->ctx->device);
        (void)hipStreamSynchronize(t->ctx->stream);
        if (t->mem) (void)hipFree(t->mem);
        forget(t->ctx->tables, t);
    }
    delete t;
    return SH_OK;
}

int sh_q4_rows(sh_ctx* c, const sh_q4* t, const int32_t* ids, int n, float* out) {
    if (!c || !t || !ids || !out || n < 1) return fail(SH_E_ARG, "sh_q4_rows: bad argument");
    if (t->ctx != c) return fail(SH_E_STATE, "sh_q4_rows: table belongs to another context");
    for (int i = 0; i < n; i++)
        if (ids[i] < 0 || ids[i] >= t->t.rows) return fail(SH_E_ARG, "sh_q4_rows: row id out of range");
    HIPCHK(hipSetDevice(c->device));
    int32_t* dids = nullptr;
    float* dout = nullptr;
    HIPCHK(hipMalloc((void**)&dids, sizeof(int32_t) * n));
    hipError_t e = hipMalloc((void**)&dout, sizeof(float) * (size_t)n * t->t.cols);
    if (e == hipSuccess) e = hipMemcpyAsync(dids, ids, sizeof(int32_t) * n, hipMemcpyHostToDevice, c->stream);
    if (e == hipSuccess) e = launch_q4_rows(t->t, dids, n, dout, c->stream);
    if (e == hipSuccess) e = hipMemcpyAsync(out, dout, sizeof(float) * (size_t)n * t->t.cols, hipMemcpyDeviceToHost, c->stream);
    if (e == hipSuccess) e = hipStreamSynchronize(c->stream);
    (void)hipFree(dids);
    if (dout) (void)hipFree(dout);
    if (e != hipSuccess) return fail(SH_E_HIP, std::string("sh_q4_rows: ") + hipGetErrorString(e));
    return SH_OK;
}

namespace {
// the kernel-level GEMV launch; with t0/t1 the launch records them around the kernel itself
int q4_gemv_launch(sh_ctx* c, const sh_q4* t, const float* x, int n_in, float* y, int cut_mode, hipEvent_t t0, hipEvent_t t1) {
    if (!c || !t || !x || !y || n_in < 1 || n_in > 2 || cut_mode < 0 || cut_mode > 1) return fail(SH_E_ARG, "sh_q4_gemv: bad argument");
    if (t->ctx != c) return fail(SH_E_STATE, "sh_q4_gemv: table belongs to another context");
    if (cut_mode == 1 && n_in != 1) return fail(SH_E_ARG, "sh_q4_gemv: the half-away cut takes one input");
    gemv_args a{};
    a.W = t->t;
    a.units = t->t.rows / 8;
    a.src = x;
    a.src_ld = t->t.cols;
    a.out = y;
    a.out_ld = t->t.rows;
    const int grid = a.units < 4096 ? a.units : 4096;
    HIPCHK(launch_gemv(n_in, cut_mode ? PRO_CUT_HALF_AWAY : PRO_CUT, EPI_STORE, grid, a, c->stream, t0, t1));
    return SH_OK;
}
}  // namespace

int sh_q4_gemv_dev(sh_ctx* c, const sh_q4* t, const float* x, int n_in, float* y, int cut_mode) {
    return q4_gemv_launch(c, t, x, n_in, y, cut_mode, nullptr, nullptr);
}

int sh_q4_gemv(sh_ctx* c, const sh_q4* t, const float* x, int n_in, float* y, int cut_mode) {
    if (!c || !t || !x || !y || n_in < 1 || n_in > 2) return fail(SH_E_ARG, "sh_q4_gemv: bad argument");
    HIPCHK(hipSetDevice(c->device));
    const size_t nx = (size_t)n_in * t->t.cols, ny = (size_t)n_in * t->t.rows;
    const size_t need = nx > ny ? nx : ny;
    if (c->bench_cap < need) {
        HIPCHK(regrow2(&c->bench_x, &c->bench_y, need));
        c->bench_cap = need;
    }
    HIPCHK(hipMemcpyAsync(c->bench_x, x, nx * 4, hipMemcpyHostToDevice, c->stream));
    const int rc = sh_q4_gemv_dev(c, t, c->bench_x, n_in, c->bench_y, cut_mode);
    if (rc != SH_OK) return rc;
    HIPCHK(hipMemcpyAsync(y, c->bench_y, ny * 4, hipMemcpyDeviceToHost, c->stream));
    HIPCHK(hipStreamSynchronize(c->stream));
    return SH_OK;
}

namespace {
// the tables (Q4_0, as sh_q4_create makes them) in launches of up to GEMV_GROUP_MAX tables (one width per launch
// for two inputs)
int q4_group_launch(sh_ctx* c, int n, sh_q4* const* t, const float* const* x, float* const* y, int n_in, int cut_mode) {
    if (!c || n < 1 || !t || !x || !y || n_in < 1 || n_in > 2 || cut_mode < 0 || cut_mode > 1 || (cut_mode == 1 && n_in != 1))
        return fail(SH_E_ARG, "sh_q4_gemv_group: bad argument");
    for (int i = 0; i < n; i++) {
        if (!t[i] || !x[i] || !y[i]) return fail(SH_E_ARG, "sh_q4_gemv_group: null table or buffer");
        if (t[i]->ctx != c) return fail(SH_E_STATE, "sh_q4_gemv_group: table belongs to another context");
        const int nb = t[i]->t.nb;
        if (nb != 64 && nb != 128 && nb != 256) return fail(SH_E_SHAPE, "sh_q4_gemv_group: cols must be 2048, 4096 or 8192");
    }
    // the widest tables first within a launch: their workgroups are the longest, so they start first
    std::vector<int> order(n);
    for (int i = 0; i < n; i++) order[i] = i;
    std::stable_sort(order.begin(), order.end(), [&](int a, int b) { return t[a]->t.nb > t[b]->t.nb; });
    std::vector<char> done(n, 0);
    for (int oi = 0; oi < n; oi++) {
        const int i = order[oi];
        if (done[i]) continue;
        gemv_group_args g{};
        g.start[0] = 0;
        for (int oj = oi; oj < n && g.n < GEMV_GROUP_MAX; oj++) {
            const int j = order[oj];
            if (done[j]) continue;
            if (n_in == 2 && t[j]->t.nb != t[i]->t.nb) continue;   // measured: two inputs run faster one width per launch
            g.W[g.n] = t[j]->t;
            g.src[g.n] = x[j];
            g.out[g.n] = y[j];
            g.start[g.n + 1] = g.start[g.n] + t[j]->t.rows / 8;
            g.n++;
            done[j] = 1;
        }
        HIPCHK(launch_gemv_group(n_in, cut_mode == 1, g, c->stream));
    }
    return SH_OK;
}
}  // namespace

int sh_q4_gemv_group_dev(sh_ctx* c, int n, sh_q4* const* tables, const float* const* x_dev, float* const* y_dev, int n_in,
                         int cut_mode) {
    if (!c) return fail(SH_E_ARG, "sh_q4_gemv_group_dev: bad argument");
    HIPCHK(hipSetDevice(c->device));
    return q4_group_launch(c, n, tables, x_dev, y_dev, n_in, cut_mode);
}

int sh_q4_gemv_group(sh_ctx* c, int n, sh_q4* const* tables, const float* const* x, float* const* y, int n_in, int cut_mode) {
    if (!c || n < 1 || !tables || !x || !y || n_in < 1 || n_in > 2) return fail(SH_E_ARG, "sh_q4_gemv_group: bad argument");
    for (int i = 0; i < n; i++)
        if (!tables[i] || !x[i] || !y[i]) return fail(SH_E_ARG, "sh_q4_gemv_group: null table or buffer");
    HIPCHK(hipSetDevice(c->device));
    size_t total = 0;
    std::vector<size_t> xo(n), yo(n);
    for (int i = 0; i < n; i++) {
        xo[i] = total;
        total += (size_t)n_in * tables[i]->t.cols;
        yo[i] = total;
        total += (size_t)n_in * tables[i]->t.rows;
    }
    float* buf = nullptr;
    HIPCHK(hipMalloc(&buf, total * sizeof(float)));
    std::vector<const float*> dx(n);
    std::vector<float*> dy(n);
    hipError_t e = hipSuccess;
    for (int i = 0; i < n && e == hipSuccess; i++) {
        dx[i] = buf + xo[i];
        dy[i] = buf + yo[i];
        e = hipMemcpyAsync(buf + xo[i], x[i], sizeof(float) * n_in * tables[i]->t.cols, hipMemcpyHostToDevice, c->stream);
    }
    int rc = e == hipSuccess ? q4_group_launch(c, n, tables, dx.data(), dy.data(), n_in, cut_mode) : SH_E_HIP;
    for (int i = 0; i < n && rc == SH_OK && e == hipSuccess; i++)
        e = hipMemcpyAsync(y[i], dy[i], sizeof(float) * n_in * tables[i]->t.rows, hipMemcpyDeviceToHost, c->stream);
    const hipError_t es = hipStreamSynchronize(c->stream);
    (void)hipFree(buf);
    if (rc != SH_OK) return rc;
    if (e != hipSuccess || es != hipSuccess)
        return fail(SH_E_HIP, std::string("sh_q4_gemv_group: ") + hipGetErrorString(e != hipSuccess ? e : es));
    return SH_OK;
}

int sh_q4_group_bench(sh_ctx* c, int n_sets, int n, sh_q4* const* tables, int n_in, int cut_mode, int reps, double* avg_us) {
    if (!c || n_sets < 1 || n < 1 || !tables || reps < 1 || n_in < 1 || n_in > 2) return fail(SH_E_ARG, "sh_q4_group_bench: bad argument");
    HIPCHK(hipSetDevice(c->device));
    size_t need = 0;   // every table of a set reads its own slice of the input buffer and writes its own output slice
    size_t xo = 0, yo = 0;
    for (int i = 0; i < n; i++) {
        xo += (size_t)n_in * tables[i]->t.cols;
        yo += (size_t)n_in * tables[i]->t.rows;
    }
    need = xo > yo ? xo : yo;
    if (c->bench_cap < need) {
        HIPCHK(regrow2(&c->bench_x, &c->bench_y, need));
        HIPCHK(hipMemset(c->bench_x, 0, need * 4));
        c->bench_cap = need;
    }
    std::vector<const float*> dx(n);
    std::vector<float*> dy(n);
    xo = yo = 0;
    for (int i = 0; i < n; i++) {
        dx[i] = c->bench_x + xo;
        dy[i] = c->bench_y + yo;
        xo += (size_t)n_in * tables[i]->t.cols;
        yo += (size_t)n_in * tables[i]->t.rows;
    }
    for (int s = 0; s < n_sets; s++) {   // warm-up: one pass over every set
        const int rc = q4_group_launch(c, n, tables + (size_t)s * n, dx.data(), dy.data(), n_in, cut_mode);
        if (rc != SH_OK) return rc;
    }
    HIPCHK(hipEventRecord(c->ev0, c->stream));
    for (int r = 0; r < reps; r++) {
        const int rc = q4_group_launch(c, n, tables + (size_t)(r % n_sets) * n, dx.data(), dy.data(), n_in, cut_mode);
        if (rc != SH_OK) return rc;
    }
    HIPCHK(hipEventRecord(c->ev1, c->stream));
    HIPCHK(hipEventSynchronize(c->ev1));
    float ms;
    HIPCHK(hipEventElapsedTime(&ms, c->ev0, c->ev1));
    if (avg_us) *avg_us = ms * 1e3 / reps;
    return SH_OK;
}

int sh_q4_bench(sh_ctx* c, sh_q4* const* tables, int n_tables, int n_in, int cut_mode, int reps, double* avg_us) {
    if (!c || !tables || n_tables < 1 || reps < 1) return fail(SH_E_ARG, "sh_q4_bench: bad argument");
    HIPCHK(hipSetDevice(c->device));
    size_t need = 0;
    for (int i = 0; i < n_tables; i++) {
        const size_t n = (size_t)n_in * (tables[i]->t.cols > tables[i]->t.rows ? tables[i]->t.cols : tables[i]->t.rows);
        need = n > need ? n : need;
    }
    if (c->bench_cap < need) {
        HIPCHK(regrow2(&c->bench_x, &c->bench_y, need));
        HIPCHK(hipMemset(c->bench_x, 0, need * 4));
        c->bench_cap = need;
    }
    for (int i = 0; i < n_tables; i++) {   // warm-up: one pass over every table
        const int rc = sh_q4_gemv_dev(c, tables[i], c->bench_x, n_in, c->bench_y, cut_mode);
        if (rc != SH_OK) return rc;
    }
    HIPCHK(hipEventRecord(c->ev0, c->stream));
    for (int r = 0; r < reps; r++) {
        const int rc = sh_q4_gemv_dev(c, tables[r % n_tables], c->bench_x, n_in, c->bench_y, cut_mode);
        if (rc != SH_OK) return rc;
    }
    HIPCHK(hipEventRecord(c->ev1, c->stream));
    HIPCHK(hipEventSynchronize(c->ev1));
    float ms;
    HIPCHK(hipEventElapsedTime(&ms, c->ev0, c->ev1));
    if (avg_us) *avg_us = ms * 1e3 / reps;
    return SH_OK;
}

int sh_q4_bench_graph(sh_ctx* c, sh_q4* const* tables, int n_tables, int n_in, int cut_mode, int passes, double* avg_us) {
    if (!c || !tables || n_tables < 1 || passes < 1) return fail(SH_E_ARG, "sh_q4_bench_graph: bad argument");
    HIPCHK(hipSetDevice(c->device));
    for (int i = 0; i < n_tables; i++) {
        const size_t need = (size_t)n_in * (tables[i]->t.cols > tables[i]->t.rows ? tables[i]->t.cols : tables[i]->t.rows);
        if (c->bench_cap < need) return fail(SH_E_STATE, "sh_q4_bench_graph: run sh_q4_bench on these tables first");
    }
    // one pass over the tables, captured once: every launch a graph node behind the one before it
    hipGraph_t graph = nullptr;
    hipGraphExec_t exec = nullptr;
    HIPCHK(hipStreamBeginCapture(c->stream, hipStreamCaptureModeThreadLocal));
    int rc = SH_OK;
    for (int i = 0; i < n_tables && rc == SH_OK; i++) rc = q4_gemv_launch(c, tables[i], c->bench_x, n_in, c->bench_y, cut_mode, nullptr, nullptr);
    hipError_t e = hipStreamEndCapture(c->stream, &graph);
    if (rc != SH_OK || e != hipSuccess) {
        if (graph) (void)hipGraphDestroy(graph);
        return rc != SH_OK ? rc : fail(SH_E_HIP, std::string("sh_q4_bench_graph: capture: ") + hipGetErrorString(e));
    }
    e = hipGraphInstantiate(&exec, graph, nullptr, nullptr, 0);
    (void)hipGraphDestroy(graph);
    if (e != hipSuccess) return fail(SH_E_HIP, std::string("sh_q4_bench_graph: instantiate: ") + hipGetErrorString(e));
    float ms = 0;
    e = hipGraphLaunch(exec, c->stream);   // warm-up pass
    if (e == hipSuccess) e = hipEventRecord(c->ev0, c->stream);
    for (int p = 0; p < passes && e == hipSuccess; p++) e = hipGraphLaunch(exec, c->stream);
    if (e == hipSuccess) e = hipEventRecord(c->ev1, c->stream);
    if (e == hipSuccess) e = hipEventSynchronize(c->ev1);
    if (e == hipSuccess) e = hipEventElapsedTime(&ms, c->ev0, c->ev1);
    (void)hipGraphExecDestroy(exec);
    if (e != hipSuccess) return fail(SH_E_HIP, std::string("sh_q4_bench_graph: ") + hipGetErrorString(e));
    if (avg_us) *avg_us = ms * 1e3 / ((double)passes * n_tables);
    return SH_OK;
}

int sh_q4_bench_kernel(sh_ctx* c, sh_q4* const* tables, int n_tables, int n_in, int cut_mode, int reps, double* avg_us) {
    if (!c || !tables || n_tables < 1 || reps < 1) return fail(SH_E_ARG, "sh_q4_bench_kernel: bad argument");
    HIPCHK(hipSetDevice(c->device));
    double total_ms = 0.0;
    for (int r = -n_tables; r < reps; r++) {   // the first pass over the tables is a warm-up
        sh_q4* t = tables[(r + n_tables) % n_tables];
        const size_t need = (size_t)n_in * (t->t.cols > t->t.rows ? t->t.cols : t->t.rows);
        if (c->bench_cap < need) return fail(SH_E_STATE, "sh_q4_bench_kernel: run sh_q4_bench on these tables first");
        const int rc = q4_gemv_launch(c, t, c->bench_x, n_in, c->bench_y, cut_mode, c->ev0, c->ev1);
        if (rc != SH_OK) return rc;
        HIPCHK(hipEventSynchronize(c->ev1));
        float ms;
        HIPCHK(hipEventElapsedTime(&ms, c->ev0, c->ev1));
        if (r >= 0) total_ms += ms;
    }
    if (avg_us) *avg_us = total_ms * 1e3 / reps;
    return SH_OK;
}

int sh_expf(sh_ctx* c, const float* x, long long n, float* y) {
    if (!c || !x || !y || n < 1) return fail(SH_E_ARG, "sh_expf: bad argument");
    HIPCHK(hipSetDevice(c->device));
    float *dx = nullptr, *dy = nullptr;
    HIPCHK(hipMalloc((void**)&dx, sizeof(float) * n));
    hipError_t e = hipMalloc((void**)&dy, sizeof(float) * n);
    if (e == hipSuccess) e = hipMemcpyAsync(dx, x, sizeof(float) * n, hipMemcpyHostToDevice, c->stream);
    if (e == hipSuccess) e = launch_expf(dx, dy, n, c->stream);
    if (e == hipSuccess) e = hipMemcpyAsync(y, dy, sizeof(float) * n, hipMemcpyDeviceToHost, c->stream);
    if (e == hipSuccess) e = hipStreamSynchronize(c->stream);
    (void)hipFree(dx);
    if (dy) (void)hipFree(dy);
    if (e != hipSuccess) return fail(SH_E_HIP, std::string("sh_expf: ") + hipGetErrorString(e));
    return SH_OK;
}

int sh_sync(sh_ctx* c) {
    if (!c) return fail(SH_E_ARG, "sh_sync: null");
    HIPCHK(hipStreamSynchronize(c->stream));
    return SH_OK;
}

}  // extern "C"
