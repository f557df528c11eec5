// Host side of the prefill (imi_seoul::step_batch, imi/core/seoul.cpp:490-655): n positions of one conversation
// through every layer at once, the table reads on the int8 matrix cores (sh_prefill.hip), then the last position's
// word scores with the step's own vocab kernel. Also the kernel-level batch product sh_q4_gemm.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdio>
#include <string>

#include "sh_ctx.h"
#include "sh_prefill.h"

using namespace sh;

namespace {
#define PCHK(x)                                                                                                \
    do {                                                                                                       \
        hipError_t e_ = (x);                                                                                   \
        if (e_ != hipSuccess) return set_error(SH_E_HIP, std::string(#x) + ": " + hipGetErrorString(e_));      \
    } while (0)

// work buffers for PF_MAX_N positions, made on first use
int prefill_buffers(sh_ctx* c) {
    if (c->pf_mem) return SH_OK;
    const sh_model_info& I = c->info;
    const size_t N = PF_MAX_N, E = I.n_embd, Hq = (size_t)I.n_head * I.head_dim;
    const size_t big = std::max<size_t>(3 * E, c->nqkv), kmax = std::max<size_t>({E, (size_t)I.n_ff, Hq});
    size_t off = 0;
    auto room = [&](size_t bytes) { const size_t at = off; off += (bytes + 255) / 256 * 256; return at; };
    const size_t o_x = room(N * E * 4), o_y = room(N * E * 4), o_big = room(N * big * 4), o_act = room(N * I.n_ff * 4);
    const size_t o_hid = room(N * E * 4), o_q = room(N * kmax), o_d = room(N * kmax / 32 * 4), o_s = room(N * kmax / 32 * 4);
    const size_t o_tok = room(N * 4), o_emb = room(N * E * 4);
    char* m = nullptr;
    PCHK(hipMalloc((void**)&m, off));
    c->pf_mem = m;
    c->pf_x = (float*)(m + o_x);
    c->pf_y = (float*)(m + o_y);
    c->pf_big = (float*)(m + o_big);
    c->pf_act = (float*)(m + o_act);
    c->pf_hid = (float*)(m + o_hid);
    c->pf_q = (int8_t*)(m + o_q);
    c->pf_d = (float*)(m + o_d);
    c->pf_s = (float*)(m + o_s);
    c->pf_tok = (int32_t*)(m + o_tok);
    c->pf_emb = (float*)(m + o_emb);
    return SH_OK;
}

// one chunk of m <= PF_MAX_N positions starting at the state's position
// the word scores' workgroups for the prefill's last position (the decode step's kernel and grid)
int prefill_scores_grid(sh_ctx* c, const gemv_args& v) {
    return c->vocab6.codes ? SH_Q6K_GRID : gemv_logits_grid(1, PRO_RESID_NORM, v, c->vocab_grid);
}

gemv_args prefill_scores_args(sh_ctx* c, const layer_dev& last, int m) {
    const int E = c->info.n_embd;
    gemv_args v{};
    v.P = c->P_dev;
    v.E = E;
    v.eps = c->eps;
    v.x_in = c->pf_x + (size_t)(m - 1) * E;   // (x before the last FFN residual: the kernel adds it itself)
    v.y_in = c->pf_y + (size_t)(m - 1) * E;
    v.w_post = last.post_ffn_norm;
    v.w_pre = c->out_norm;
    v.W = c->vocab;
    v.W6 = c->vocab6;
    v.units = c->vocab.rows / 8;
    v.out = c->logits;
    v.out_ld = c->info.n_vocab;
    v.part_v = c->part_v;
    v.part_i = c->part_i;
    return v;
}

// scores: the last position's word scores with the decode step's kernel (its prologue forms the output norm of the
// last FFN residual itself), launched before the last rows kernel updates x in place
int enqueue_chunk(sh_ctx* c, sh_state* st, int m, bool have_tokens, bool have_embd, bool scores) {
    const sh_model_info& I = c->info;
    const int E = I.n_embd, D = I.head_dim, Hq = I.n_head * D;
    hipStream_t s = c->stream;
    const pf_cut cut{c->pf_q, c->pf_d, c->pf_s};
    pf_rows_args r{};
    r.n = m;
    r.E = E;
    r.eps = c->eps;
    r.tokens = have_tokens ? c->pf_tok : nullptr;
    r.embd = have_embd ? c->pf_emb : nullptr;
    r.vocab = c->vocab;
    r.vocab6 = c->vocab6;
    r.x = c->pf_x;
    r.w_pre = c->layers[0].attn_norm;
    r.cut = cut;
    PCHK(launch_pf_rows(PFR_FIRST, r, s));
    auto gemm = [&](const q4dev& W, int epi, float* out, int ld, const pf_cut& in) {
        pf_gemm_args g{};
        g.W = W;
        g.n = m;
        g.in = in;
        g.out = out;
        g.out_ld = ld;
        return launch_pf_gemm(epi, g, s);
    };
    // the FFN activations' cut, written by the gate|up products themselves into the activation buffer's space (their
    // input cut is still being read meanwhile, so not the shared cut buffer)
    const size_t nact = (size_t)PF_MAX_N * I.n_ff;
    const pf_cut act_cut{(int8_t*)c->pf_act, (float*)((char*)c->pf_act + nact), (float*)((char*)c->pf_act + nact + nact / 8)};
    for (size_t il = 0; il < c->layers.size(); il++) {
        const layer_dev& L = c->layers[il];
        pf_conv_args cv{};   // (a conv layer: its memory update rides on the next rows launch)
        if (L.conv) {
            PCHK(gemm(L.in_proj, EPI_STORE, c->pf_big, 3 * E, cut));
            cv.bcx = c->pf_big;
            cv.w = L.conv_w;
            cv.state = st->conv + (size_t)L.ci * I.d_conv * E;
            cv.n = m;
            cv.E = E;
            cv.d_conv = I.d_conv;
            cv.cut = cut;
            PCHK(launch_pf_conv_lanes(cv, s));
            PCHK(gemm(L.out_proj, EPI_STORE, c->pf_y, E, cut));
        } else {
            PCHK(gemm(L.qkvg, EPI_STORE, c->pf_big, c->nqkv, cut));
            pf_attn_args t{};
            t.qkv = c->pf_big;
            t.ld = c->nqkv;
            t.q_norm = L.q_norm;
            t.k_norm = L.k_norm;
            t.rope_cs = L.swa ? c->rope_cs_swa : c->rope_cs;
            t.kc = st->kc + (size_t)L.ai * I.n_head_kv * I.n_ctx * D;
            t.vc = st->vc + (size_t)L.ai * I.n_head_kv * I.n_ctx * D;
            t.n = m;
            t.pos0 = st->pos;
            t.n_head = I.n_head;
            t.n_kv = I.n_head_kv;
            t.D = D;
            t.n_ctx = I.n_ctx;
            t.n_swa = L.swa ? I.n_swa : 0;
            t.eps = c->eps;
            t.cut = cut;
            PCHK(launch_pf_kv(t, s));
            PCHK(launch_pf_attn(t, s));
            PCHK(gemm(L.o, EPI_STORE, c->pf_y, E, cut));
        }
        pf_rows_args f = r;
        f.conv = cv;
        f.w_post = L.post_attn_norm;
        f.y = c->pf_y;
        f.w_pre = L.ffn_norm;
        PCHK(launch_pf_rows(PFR_RESID, f, s));
        pf_gemm_args gu{};
        gu.W = L.gate_up;
        gu.n = m;
        gu.in = cut;
        gu.out_ld = I.n_ff;
        gu.outc = act_cut;
        if (pf_swiglu_cut_takes(gu)) {   // SwiGLU and the cut in the products' epilogue
            PCHK(launch_pf_gemm(EPI_SWIGLU, gu, s));
            PCHK(gemm(L.down, EPI_STORE, c->pf_y, E, act_cut));
        } else {
            PCHK(gemm(L.gate_up, EPI_SWIGLU, c->pf_act, I.n_ff, cut));
            pf_cutk_args ck{c->pf_act, I.n_ff, I.n_ff, m, cut};
            PCHK(launch_pf_cut(ck, s));
            PCHK(gemm(L.down, EPI_STORE, c->pf_y, E, cut));
        }
        pf_rows_args z = r;
        z.y = c->pf_y;
        z.w_post = L.post_ffn_norm;
        if (scores && il + 1 == c->layers.size()) {
            const gemv_args v = prefill_scores_args(c, L, m);
            const int grid = prefill_scores_grid(c, v);
            if (c->vocab6.codes) PCHK(launch_scores_q6k(1, grid, v, s));
            else PCHK(launch_gemv(1, PRO_RESID_NORM, EPI_LOGITS, grid, v, s));
        }
        if (il + 1 < c->layers.size()) {
            z.w_pre = c->layers[il + 1].attn_norm;
        } else {   // the output norm: hidden rows, no cut
            z.w_pre = c->out_norm;
            z.cut = pf_cut{};
            z.hidden = c->pf_hid;
        }
        PCHK(launch_pf_rows(PFR_RESID, z, s));
    }
    return SH_OK;
}
}  // namespace

namespace sh {
// imi_seoul::step_batch on the device. tokens[n] and/or embd[n][E] are host arrays (a position whose token is < 0,
// or every position when tokens is null, reads its embd row). The whole batch must fit the context (else nothing
// is stepped). hidden_last / logits / best get the last position's hidden state, word scores and their first
// maximum; hidden_all[n][E] every position's hidden state.
int run_prefill(sh_ctx* c, sh_state* st, const int32_t* tokens, const float* embd, int n, bool want_logits,
                float* hidden_last, float* logits, float* hidden_all, int32_t* best) {
    const sh_model_info& I = c->info;
    const int E = I.n_embd;
    if (st->pos + n > I.n_ctx) {
        fprintf(stderr, "seoul-hip: context full (%d)\n", I.n_ctx);
        return set_error(SH_E_CONTEXT_FULL, "sh_step_batch: context full");
    }
    if (tokens)
        for (int i = 0; i < n; i++)
            if (tokens[i] >= I.n_vocab || (tokens[i] < 0 && !embd)) return set_error(SH_E_ARG, "sh_step_batch: token out of range");
    PCHK(hipSetDevice(c->device));
    const int rc0 = prefill_buffers(c);
    if (rc0 != SH_OK) return rc0;
    int last_m = 0;
    for (int i0 = 0; i0 < n; i0 += PF_MAX_N) {
        const int m = std::min(PF_MAX_N, n - i0);
        if (tokens) PCHK(hipMemcpyAsync(c->pf_tok, tokens + i0, (size_t)m * 4, hipMemcpyHostToDevice, c->stream));
        if (embd) PCHK(hipMemcpyAsync(c->pf_emb, embd + (size_t)i0 * E, (size_t)m * E * 4, hipMemcpyHostToDevice, c->stream));
        const int rc = enqueue_chunk(c, st, m, tokens != nullptr, embd != nullptr, want_logits && i0 + m == n);
        if (rc != SH_OK) return rc;
        if (hidden_all) PCHK(hipMemcpyAsync(hidden_all + (size_t)i0 * E, c->pf_hid, (size_t)m * E * 4, hipMemcpyDeviceToHost, c->stream));
        // the host arrays of this chunk are read before the next chunk's copies overwrite the device buffers
        PCHK(hipStreamSynchronize(c->stream));
        st->pos += m;
        last_m = m;
    }
    const float* hl = c->pf_hid + (size_t)(last_m - 1) * E;
    if (hidden_last) PCHK(hipMemcpyAsync(hidden_last, hl, (size_t)E * 4, hipMemcpyDeviceToHost, c->stream));
    int32_t b = -1;
    if (want_logits) {   // (the scores themselves were launched in the last chunk)
        const int grid = prefill_scores_grid(c, prefill_scores_args(c, c->layers.back(), last_m));
        final_args z{};
        z.E = E;
        z.eps = c->eps;
        z.part_v = c->part_v;
        z.part_i = c->part_i;
        z.n_part = grid;
        z.logits = c->logits;
        z.ld_logits = I.n_vocab;
        z.P = c->P_dev;
        z.advance = 0;
        PCHK(launch_final(1, z, c->stream));
        if (logits) PCHK(hipMemcpyAsync(logits, c->logits, (size_t)I.n_vocab * 4, hipMemcpyDeviceToHost, c->stream));
        PCHK(hipMemcpyAsync(&b, &c->P_dev->best[0], 4, hipMemcpyDeviceToHost, c->stream));
    }
    PCHK(hipStreamSynchronize(c->stream));
    if (best) *best = b;
    return SH_OK;
}
}  // namespace sh

extern "C" int sh_q4_gemm(sh_ctx* c, const sh_q4* t, const float* x, int n, float* y) {
    if (!c || !t || !x || !y || n < 1 || n > PF_MAX_N) return set_error(SH_E_ARG, "sh_q4_gemm: bad argument (1 <= n <= 512)");
    if (t->ctx != c) return set_error(SH_E_STATE, "sh_q4_gemm: table belongs to another context");
    PCHK(hipSetDevice(c->device));
    const q4dev& W = t->t;
    const size_t nx = (size_t)n * W.cols, ny = (size_t)n * W.rows;
    char* m = nullptr;
    const size_t o_y = (nx * 4 + 255) / 256 * 256, o_q = o_y + (ny * 4 + 255) / 256 * 256;
    const size_t o_d = o_q + (nx + 255) / 256 * 256, o_s = o_d + (nx / 32 * 4 + 255) / 256 * 256;
    PCHK(hipMalloc((void**)&m, o_s + nx / 32 * 4));
    const pf_cut cut{(int8_t*)(m + o_q), (float*)(m + o_d), (float*)(m + o_s)};
    hipError_t e = hipMemcpyAsync(m, x, nx * 4, hipMemcpyHostToDevice, c->stream);
    if (e == hipSuccess) e = launch_pf_cut(pf_cutk_args{(const float*)m, W.cols, W.cols, n, cut}, c->stream);
    pf_gemm_args g{};
    g.W = W;
    g.n = n;
    g.in = cut;
    g.out = (float*)(m + o_y);
    g.out_ld = W.rows;
    if (e == hipSuccess) e = launch_pf_gemm(EPI_STORE, g, c->stream);
    if (e == hipSuccess) e = hipMemcpyAsync(y, m + o_y, ny * 4, hipMemcpyDeviceToHost, c->stream);
    if (e == hipSuccess) e = hipStreamSynchronize(c->stream);
    (void)hipFree(m);
    if (e != hipSuccess) return set_error(SH_E_HIP, std::string("sh_q4_gemm: ") + hipGetErrorString(e));
    return SH_OK;
}
