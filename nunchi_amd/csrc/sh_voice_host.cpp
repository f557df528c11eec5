// Host side of the Q8_0 voice generator (imi_voice, imi/core/voice.{h,cpp}) behind the C ABI of
// include/seoul_hip.h: GGUF read, repack of every 8-bit table into the device layout of sh_voice.h, the frame's
// input projection, masked passes (replayed from a captured HIP graph), and the feedback row sum.
#include "../../include/seoul_hip.h"

#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstddef>
#include <cstdlib>
#include <cstring>
#include <string>
#include <vector>

#include "gguf_file.h"
#include "sh_voice.h"

namespace sh {
int set_error(int code, const std::string& msg);   // sh_engine.cpp: the thread's last error message
}
using namespace sh;

namespace {
#define VCHK(x)                                                                                                 \
    do {                                                                                                        \
        hipError_t e_ = (x);                                                                                    \
        if (e_ != hipSuccess) return set_error(SH_E_HIP, std::string(#x) + ": " + hipGetErrorString(e_));       \
    } while (0)

}  // namespace

// Q8_0 rows (pointers to n_cols / 32 blocks of fp16 d + 32 int8 each) -> codes [G][nb][8][32], scales [G][nb][8]
// (the grouping of imi_q8g::build, imi/core/tables.cpp:297-318, with the 32 codes of a block kept together)
void sh::repack_q8(const std::vector<const uint8_t*>& rows, int cols, std::vector<int8_t>& codes, std::vector<uint16_t>& scales) {
    const int R = (int)rows.size(), G = (R + 7) / 8, nb = cols / 32;
    codes.assign((size_t)G * nb * 8 * 32, 0);
    scales.assign((size_t)G * nb * 8, 0);
    for (int r = 0; r < R; r++)
        for (int j = 0; j < nb; j++) {
            const uint8_t* b = rows[r] + (size_t)j * 34;
            const size_t blk = ((size_t)(r / 8) * nb + j) * 8 + (r % 8);
            memcpy(&scales[blk], b, 2);
            memcpy(&codes[blk * 32], b + 2, 32);
        }
}

namespace {

struct vlayer {
    q8dev qkvg, o, gate_up, down;
    const float *ln1 = nullptr, *ln2 = nullptr, *q_norm = nullptr, *k_norm = nullptr;
};

struct pass_in {               // one host -> device copy per pass
    int32_t n_need;
    int32_t codes[VX_MAX_P];
    int32_t need[VX_MAX_P];
};

struct sample_io {             // the sampler's inputs (host -> device) and outputs (device -> host)
    double u[VX_MAX_P];
    double keep[VX_MAX_P];
    int32_t picks[VX_MAX_P];
    int32_t hist[VS_MAX_HIST * VX_MAX_P];   // only the frames given are copied
};
}  // namespace

struct sh_voice {
    int device = 0;
    hipStream_t stream = nullptr;
    sh_voice_shape info{};
    float eps = 1e-5f, rope_theta = 1e6f;
    int n_qkv = 0;
    char* mem = nullptr;               // every table, norm and buffer, one allocation
    std::vector<vlayer> layers;
    q8dev* tabs_dev = nullptr;         // [n_cb] score tables, then [1] the input projection
    const float *proj_b = nullptr, *mask = nullptr, *out_norm = nullptr, *head_norm = nullptr;
    const uint8_t* feed_rows = nullptr;
    long long feed_row_bytes = 0;
    const float2* rope_cs = nullptr;
    float *x = nullptr, *qkv = nullptr, *att = nullptr, *act = nullptr, *base = nullptr, *hid = nullptr;
    float *out = nullptr, *fb = nullptr;
    float* part = nullptr;             // per-block sums of the o and down tables split over column chunks
    pass_in* in_dev = nullptr;
    pass_in* in_host = nullptr;        // pinned
    sample_io* smp_dev = nullptr;
    sample_io* smp_host = nullptr;     // pinned
    int last_need = -1;                // codebooks the last pass scored (-1: no pass since the frame began)
    bool use_graph = true;
    hipGraphExec_t graph = nullptr;
};

namespace {
// workgroups of a pass table: one per row group in the generic order, one per two groups in the scaled order
// (and per gate|up group pair, in both)
int units_of(int P, const q8dev& W) {
    const int G = W.rows_pad / 8;
    return (P == 6 || P == 12) ? (G + 1) / 2 : G;
}

int enqueue_pass(sh_voice* v) {
    const sh_voice_shape& I = v->info;
    const int P = I.n_cb, E = I.n_embd, D = I.head_dim, Hq = I.n_head * D;
    vembed_args ea{v->tabs_dev, E, P, v->in_dev->codes, v->mask, v->base, v->x};
    VCHK(launch_vembed(ea, v->stream));
    for (const vlayer& L : v->layers) {
        vtab_args t{};
        t.eps = v->eps;
        t.W = L.qkvg; t.src = v->x; t.src_ld = E; t.norm_w = L.ln1; t.out = v->qkv; t.out_ld = v->n_qkv;
        t.units = units_of(P, L.qkvg);
        VCHK(launch_vtab(P, VP_NORM, VE_STORE, t, v->stream));
        vattn_args aa{v->qkv, v->n_qkv, v->att, L.q_norm, L.k_norm, v->rope_cs, P, I.n_head, I.n_head_kv, D, v->eps,
                      1.0f / sqrtf((float)D)};
        VCHK(launch_vattn(aa, v->stream));
        t = vtab_args{};
        t.eps = v->eps;
        t.W = L.o; t.src = v->att; t.src_ld = Hq; t.out = v->x; t.out_ld = E; t.part = v->part;
        t.units = units_of(P, L.o);
        VCHK(launch_vtab(P, VP_PLAIN, VE_RESID, t, v->stream));
        t = vtab_args{};
        t.eps = v->eps;
        t.W = L.gate_up; t.src = v->x; t.src_ld = E; t.norm_w = L.ln2; t.out = v->act; t.out_ld = I.n_ff;
        t.units = L.gate_up.rows_pad / 16;
        VCHK(launch_vtab(P, VP_NORM, VE_SWIGLU, t, v->stream));
        t = vtab_args{};
        t.eps = v->eps;
        t.W = L.down; t.src = v->act; t.src_ld = I.n_ff; t.out = v->x; t.out_ld = E; t.part = v->part;
        t.units = units_of(P, L.down);
        VCHK(launch_vtab(P, VP_PLAIN, VE_RESID, t, v->stream));
    }
    vone_args sa{};
    sa.tabs = v->tabs_dev; sa.rows = I.n_vocab; sa.src = v->x; sa.head = 1; sa.out_norm = v->out_norm;
    sa.head_norm = v->head_norm; sa.need = v->in_dev->need; sa.n_need = &v->in_dev->n_need; sa.eps = v->eps;
    sa.out = v->out; sa.rows_per_wg = 64;
    VCHK(launch_vone(sa, P, E, v->stream));
    return SH_OK;
}

void release(sh_voice* v) {
    if (v->graph) (void)hipGraphExecDestroy(v->graph);
    if (v->mem) (void)hipFree(v->mem);
    if (v->in_host) (void)hipHostFree(v->in_host);
    if (v->smp_host) (void)hipHostFree(v->smp_host);
    if (v->stream) (void)hipStreamDestroy(v->stream);
    delete v;
}
}  // namespace

extern "C" {

int sh_voice_load(int device, const char* path, sh_voice** out) {
    if (!path || !out) return set_error(SH_E_ARG, "sh_voice_load: bad argument");
    *out = nullptr;
    VCHK(hipSetDevice(device));
    gg_file f;
    if (!f.load(path)) return set_error(SH_E_FILE, "sh_voice_load: " + f.error);
    const std::string g = "a.gen.code.";
    const gg_tensor *embd = f.get(g + "embd.weight"), *oe = f.get(g + "out_embd.weight"), *pw = f.get(g + "proj_in.weight");
    const gg_tensor *pb = f.get(g + "proj_in.bias"), *me = f.get(g + "mask_embd"), *on = f.get(g + "output_norm.weight");
    const gg_tensor* hn = f.get(g + "head_norm.weight");
    if (!embd || !oe || !pw || !pb || !me || !on || !hn) return set_error(SH_E_FILE, "sh_voice_load: " + f.error);
    if (embd->type != GT_Q8_0 || oe->type != GT_Q8_0 || pw->type != GT_Q8_0)
        return set_error(SH_E_SHAPE, "sh_voice_load: the generator needs 8-bit (Q8_0) tables");
    sh_voice_shape I{};
    I.n_embd = (int)embd->ne[0];
    I.n_vocab = (int)embd->ne[1];
    I.n_cb = (int)embd->ne[2];
    I.n_in = (int)pw->ne[0];
    const int E = I.n_embd, P = I.n_cb;
    if (P < 2 || P > VX_MAX_P) return set_error(SH_E_SHAPE, "sh_voice_load: 2 to 12 codebooks are supported");
    if (E % 32 || E > 4096 || I.n_in % 32 || I.n_in > 4096)
        return set_error(SH_E_SHAPE, "sh_voice_load: n_embd and the input width must be multiples of 32, at most 4096");
    if (pw->ne[1] != (int64_t)P * E || oe->ne[0] != I.n_in || oe->ne[1] != (int64_t)P * I.n_vocab)
        return set_error(SH_E_SHAPE, "sh_voice_load: proj_in / out_embd shapes do not match the code tables");
    auto f32n = [&](const gg_tensor* t, int64_t n) { return t->type == GT_F32 && t->ne[0] * t->ne[1] * t->ne[2] == n; };
    if (!f32n(pb, (int64_t)P * E) || !f32n(me, E) || !f32n(on, E) || !f32n(hn, (int64_t)P * E))
        return set_error(SH_E_SHAPE, "sh_voice_load: norm / bias / mask vectors must be f32 of the model's widths");

    // tables in upload order: per layer qkvg, o, gate_up, down; then the score tables, then proj_in
    struct plan { std::vector<const uint8_t*> rows; int cols; q8dev* dst; };
    std::vector<plan> tabs;
    auto rows_of = [](std::vector<const uint8_t*>& o, const gg_tensor* t, int r0, int n, int plane) {
        for (int r = r0; r < r0 + n; r++)
            o.push_back(static_cast<const uint8_t*>(t->data) + (size_t)plane * t->nb[2] + (size_t)r * t->nb[1]);
    };
    std::vector<std::pair<const gg_tensor*, const float**>> vecs;
    std::vector<vlayer> layers;
    for (int il = 0;; il++) {
        const std::string p = g + "blk." + std::to_string(il) + ".";
        if (!f.get(p + "ln1.weight", false)) break;
        layers.emplace_back();
    }
    if (layers.empty()) return set_error(SH_E_FILE, "sh_voice_load: no generator layers");
    for (size_t il = 0; il < layers.size(); il++) {
        const std::string p = g + "blk." + std::to_string(il) + ".";
        vlayer& L = layers[il];
        const gg_tensor *q = f.get(p + "attn_q.weight"), *k = f.get(p + "attn_k.weight"), *vv = f.get(p + "attn_v.weight");
        const gg_tensor *ga = f.get(p + "attn_gate.weight"), *o = f.get(p + "attn_out.weight");
        const gg_tensor *fg = f.get(p + "ffn_gate.weight"), *fu = f.get(p + "ffn_up.weight"), *fd = f.get(p + "ffn_down.weight");
        const gg_tensor *l1 = f.get(p + "ln1.weight"), *l2 = f.get(p + "ln2.weight");
        const gg_tensor *qn = f.get(p + "attn_q_norm.weight"), *kn = f.get(p + "attn_k_norm.weight");
        if (!q || !k || !vv || !ga || !o || !fg || !fu || !fd || !l1 || !l2 || !qn || !kn)
            return set_error(SH_E_FILE, "sh_voice_load: " + f.error);
        for (const gg_tensor* t : {q, k, vv, ga, o, fg, fu, fd})
            if (t->type != GT_Q8_0) return set_error(SH_E_SHAPE, "sh_voice_load: a generator table is not Q8_0");
        const int D = (int)qn->ne[0];
        if (il == 0) {
            I.head_dim = D;
            I.n_head = (int)(q->ne[1] / D);
            I.n_head_kv = (int)(k->ne[1] / D);
            I.n_ff = (int)fg->ne[1];
        }
        if (D != I.head_dim || D > VX_MAX_D || D % 32 || I.n_head_kv < 1 || I.n_head % I.n_head_kv ||
            q->ne[1] != (int64_t)I.n_head * D || k->ne[1] != (int64_t)I.n_head_kv * D || vv->ne[1] != k->ne[1] ||
            ga->ne[1] != I.n_head || q->ne[0] != E || o->ne[1] != E || o->ne[0] != (int64_t)I.n_head * D ||
            fg->ne[1] != I.n_ff || fu->ne[1] != I.n_ff || I.n_ff % 8 || fd->ne[1] != E || fd->ne[0] != I.n_ff)
            return set_error(SH_E_SHAPE, "sh_voice_load: layer shapes not supported (head_dim 32 or 64, n_ff % 8 == 0)");
        if (!f32n(l1, E) || !f32n(l2, E) || !f32n(qn, D) || !f32n(kn, D))
            return set_error(SH_E_SHAPE, "sh_voice_load: layer norms must be f32");
        vecs.push_back({l1, &L.ln1});
        vecs.push_back({l2, &L.ln2});
        vecs.push_back({qn, &L.q_norm});
        vecs.push_back({kn, &L.k_norm});
        plan pq{{}, E, &L.qkvg};   // q | k | v | gate stacked (voice.cpp:52)
        for (const gg_tensor* t : {q, k, vv, ga}) rows_of(pq.rows, t, 0, (int)t->ne[1], 0);
        tabs.push_back(std::move(pq));
        plan po{{}, (int)o->ne[0], &L.o};
        rows_of(po.rows, o, 0, E, 0);
        tabs.push_back(std::move(po));
        plan pg{{}, E, &L.gate_up};   // gate and up interleaved by 8-row group (voice.cpp:57-59)
        for (int t = 0; t < I.n_ff; t += 8) { rows_of(pg.rows, fg, t, 8, 0); rows_of(pg.rows, fu, t, 8, 0); }
        tabs.push_back(std::move(pg));
        plan pd{{}, I.n_ff, &L.down};
        rows_of(pd.rows, fd, 0, E, 0);
        tabs.push_back(std::move(pd));
    }
    I.n_layer = (int)layers.size();
    std::vector<q8dev> tab_host(P + 1);
    for (int c = 0; c < P; c++) {
        plan ps{{}, E, &tab_host[c]};
        rows_of(ps.rows, embd, 0, I.n_vocab, c);
        tabs.push_back(std::move(ps));
    }
    {
        plan pp{{}, I.n_in, &tab_host[P]};
        rows_of(pp.rows, pw, 0, P * E, 0);
        tabs.push_back(std::move(pp));
    }
    vecs.push_back({pb, nullptr});
    vecs.push_back({me, nullptr});
    vecs.push_back({on, nullptr});
    vecs.push_back({hn, nullptr});

    auto* v = new sh_voice;
    v->device = device;
    v->info = I;
    v->layers = std::move(layers);
    v->n_qkv = (I.n_head + 2 * I.n_head_kv) * I.head_dim + I.n_head;
    v->use_graph = !(getenv("SEOUL_HIP_GRAPHS") && !strcmp(getenv("SEOUL_HIP_GRAPHS"), "0"));
    const int D = I.head_dim, Hq = I.n_head * D;

    // one device allocation: tables, vectors, feedback rows, rope table, work buffers
    size_t need = 0;
    auto room = [&](size_t n) { need += (n + 255) / 256 * 256; };
    for (const plan& t : tabs) {
        const size_t G = (t.rows.size() + 7) / 8, nb = t.cols / 32;
        room(G * nb * 256);
        room(G * nb * 16);
    }
    for (auto& vv : vecs) room((size_t)(vv.first->ne[0] * vv.first->ne[1] * vv.first->ne[2]) * 4);
    room((size_t)(P + 1) * sizeof(q8dev));
    room((size_t)oe->ne[1] * oe->nb[1]);
    room((size_t)P * (D / 2) * sizeof(float2));
    const size_t wide = (size_t)P * std::max({E, Hq, I.n_ff, v->n_qkv, I.n_vocab});
    for (int i = 0; i < 5; i++) room(wide * 4);   // x, qkv, att, act, out
    const size_t part_floats = (size_t)(E + 7) / 8 * 8 * P * (std::max(Hq, I.n_ff) / 32);
    room(part_floats * 4);
    room((size_t)P * E * 4 + I.n_in * 4 * 2);
    room(sizeof(pass_in));
    room(sizeof(sample_io));
    hipError_t e = hipStreamCreateWithFlags(&v->stream, hipStreamNonBlocking);
    if (e == hipSuccess) e = hipMalloc(&v->mem, need);
    if (e == hipSuccess) e = hipHostMalloc(reinterpret_cast<void**>(&v->in_host), sizeof(pass_in), hipHostMallocDefault);
    if (e == hipSuccess) e = hipHostMalloc(reinterpret_cast<void**>(&v->smp_host), sizeof(sample_io), hipHostMallocDefault);
    if (e != hipSuccess) {
        release(v);
        return set_error(SH_E_NOMEM, std::string("sh_voice_load: device allocation: ") + hipGetErrorString(e));
    }
    size_t used = 0;
    auto take = [&](size_t n) { char* p = v->mem + used; used += (n + 255) / 256 * 256; return p; };
    std::vector<int8_t> codes;
    std::vector<uint16_t> scales;
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
        if (e != hipSuccess) { release(v); return set_error(SH_E_HIP, std::string("sh_voice_load: upload: ") + hipGetErrorString(e)); }
        d.codes = reinterpret_cast<const int8_t*>(cp);
        d.scales = reinterpret_cast<const uint16_t*>(sp);
        *t.dst = d;
    }
    std::vector<const float*> vdev;
    for (auto& vv : vecs) {
        const size_t n = (size_t)(vv.first->ne[0] * vv.first->ne[1] * vv.first->ne[2]) * 4;
        char* p = take(n);
        e = hipMemcpy(p, vv.first->data, n, hipMemcpyHostToDevice);
        if (e != hipSuccess) { release(v); return set_error(SH_E_HIP, std::string("sh_voice_load: upload: ") + hipGetErrorString(e)); }
        if (vv.second) *vv.second = reinterpret_cast<const float*>(p);
        vdev.push_back(reinterpret_cast<const float*>(p));
    }
    const size_t nv = vdev.size();
    v->proj_b = vdev[nv - 4];
    v->mask = vdev[nv - 3];
    v->out_norm = vdev[nv - 2];
    v->head_norm = vdev[nv - 1];
    v->tabs_dev = reinterpret_cast<q8dev*>(take((size_t)(P + 1) * sizeof(q8dev)));
    char* fr = take((size_t)oe->ne[1] * oe->nb[1]);
    // rope by position (voice.cpp:11-19): th = p, multiplied by theta^(-2/D) per pair, with the C library's
    // powf / cosf / sinf, as the CPU path computes it
    std::vector<float2> rcs((size_t)P * (D / 2));
    const float rscale = powf(v->rope_theta, -2.0f / (float)D);
    for (int p = 0; p < P; p++) {
        float th = (float)p;
        for (int i = 0; i < D / 2; i++) {
            rcs[(size_t)p * (D / 2) + i] = make_float2(cosf(th), sinf(th));
            th *= rscale;
        }
    }
    char* rp = take(rcs.size() * sizeof(float2));
    e = hipMemcpy(v->tabs_dev, tab_host.data(), tab_host.size() * sizeof(q8dev), hipMemcpyHostToDevice);
    if (e == hipSuccess) e = hipMemcpy(fr, oe->data, (size_t)oe->ne[1] * oe->nb[1], hipMemcpyHostToDevice);
    if (e == hipSuccess) e = hipMemcpy(rp, rcs.data(), rcs.size() * sizeof(float2), hipMemcpyHostToDevice);
    if (e != hipSuccess) { release(v); return set_error(SH_E_HIP, std::string("sh_voice_load: upload: ") + hipGetErrorString(e)); }
    v->feed_rows = reinterpret_cast<const uint8_t*>(fr);
    v->feed_row_bytes = (long long)oe->nb[1];
    v->rope_cs = reinterpret_cast<const float2*>(rp);
    v->x = reinterpret_cast<float*>(take(wide * 4));
    v->qkv = reinterpret_cast<float*>(take(wide * 4));
    v->att = reinterpret_cast<float*>(take(wide * 4));
    v->act = reinterpret_cast<float*>(take(wide * 4));
    v->out = reinterpret_cast<float*>(take(wide * 4));
    v->part = reinterpret_cast<float*>(take(part_floats * 4));
    v->base = reinterpret_cast<float*>(take((size_t)P * E * 4 + I.n_in * 4 * 2));
    v->hid = v->base + (size_t)P * E;
    v->fb = v->hid + I.n_in;
    v->in_dev = reinterpret_cast<pass_in*>(take(sizeof(pass_in)));
    v->smp_dev = reinterpret_cast<sample_io*>(take(sizeof(sample_io)));
    if (used > need) {   // the carving above must follow the sizing pass piece by piece
        release(v);
        return set_error(SH_E_NOMEM, "sh_voice_load: internal layout error");
    }
    long long tb = 0;
    for (const plan& t : tabs) tb += (long long)((t.rows.size() + 7) / 8) * (t.cols / 32) * 8 * 34;
    v->info.table_bytes = tb;
    v->info.feedback_bytes = (long long)oe->ne[1] * oe->nb[1];
    // a frame starts from a zero base until begin_frame runs
    e = hipMemset(v->base, 0, (size_t)P * E * 4);
    if (e == hipSuccess) e = hipDeviceSynchronize();
    if (e != hipSuccess) { release(v); return set_error(SH_E_HIP, std::string("sh_voice_load: ") + hipGetErrorString(e)); }
    *out = v;
    return SH_OK;
}

int sh_voice_free(sh_voice* v) {
    if (!v) return set_error(SH_E_ARG, "sh_voice_free: null");
    (void)hipSetDevice(v->device);
    (void)hipStreamSynchronize(v->stream);
    release(v);
    return SH_OK;
}

int sh_voice_info(const sh_voice* v, sh_voice_shape* out) {
    if (!v || !out) return set_error(SH_E_ARG, "sh_voice_info: bad argument");
    *out = v->info;
    return SH_OK;
}

int sh_voice_begin_frame(sh_voice* v, const float* hidden) {
    if (!v || !hidden) return set_error(SH_E_ARG, "sh_voice_begin_frame: bad argument");
    VCHK(hipSetDevice(v->device));
    VCHK(hipMemcpyAsync(v->hid, hidden, (size_t)v->info.n_in * 4, hipMemcpyHostToDevice, v->stream));
    vone_args a{};
    a.tabs = v->tabs_dev + v->info.n_cb;
    a.rows = v->info.n_cb * v->info.n_embd;
    a.src = v->hid;
    a.bias = v->proj_b;
    a.eps = v->eps;
    a.out = v->base;
    a.rows_per_wg = 64;
    VCHK(launch_vone(a, 1, v->info.n_in, v->stream));
    VCHK(hipStreamSynchronize(v->stream));
    return SH_OK;
}

int sh_voice_base(sh_voice* v, float* out) {
    if (!v || !out) return set_error(SH_E_ARG, "sh_voice_base: bad argument");
    VCHK(hipSetDevice(v->device));
    VCHK(hipMemcpyAsync(out, v->base, (size_t)v->info.n_cb * v->info.n_embd * 4, hipMemcpyDeviceToHost, v->stream));
    VCHK(hipStreamSynchronize(v->stream));
    return SH_OK;
}

int sh_voice_pass(sh_voice* v, const int32_t* codes, const int32_t* need, int n_need, float* out) {
    if (!v || !codes || n_need < 0 || n_need > v->info.n_cb || (n_need && !need))
        return set_error(SH_E_ARG, "sh_voice_pass: bad argument (0 <= n_need <= n_cb)");
    const int P = v->info.n_cb;
    for (int i = 0; i < P; i++)
        if (codes[i] >= v->info.n_vocab) return set_error(SH_E_ARG, "sh_voice_pass: code out of range");
    for (int j = 0; j < n_need; j++)
        if (need[j] < 0 || need[j] >= P) return set_error(SH_E_ARG, "sh_voice_pass: codebook out of range");
    VCHK(hipSetDevice(v->device));
    v->last_need = -1;
    pass_in& in = *v->in_host;
    in.n_need = n_need;
    for (int i = 0; i < VX_MAX_P; i++) {
        in.codes[i] = i < P ? codes[i] : -1;
        in.need[i] = i < n_need ? need[i] : 0;
    }
    VCHK(hipMemcpyAsync(v->in_dev, &in, sizeof(pass_in), hipMemcpyHostToDevice, v->stream));
    if (v->use_graph) {
        if (!v->graph) {
            hipGraph_t gr = nullptr;
            VCHK(hipStreamBeginCapture(v->stream, hipStreamCaptureModeThreadLocal));
            const int rc = enqueue_pass(v);
            const hipError_t ec = hipStreamEndCapture(v->stream, &gr);
            if (rc != SH_OK || ec != hipSuccess) {   // (the captured graph, if any, is not kept)
                if (gr) (void)hipGraphDestroy(gr);
                if (rc != SH_OK) return rc;
                VCHK(ec);
            }
            const hipError_t ei = hipGraphInstantiate(&v->graph, gr, nullptr, nullptr, 0);
            (void)hipGraphDestroy(gr);
            VCHK(ei);
        }
        VCHK(hipGraphLaunch(v->graph, v->stream));
    } else {
        const int rc = enqueue_pass(v);
        if (rc != SH_OK) return rc;
    }
    if (out) {
        if (n_need) VCHK(hipMemcpyAsync(out, v->out, (size_t)n_need * v->info.n_vocab * 4, hipMemcpyDeviceToHost, v->stream));
        VCHK(hipStreamSynchronize(v->stream));
    }
    v->last_need = n_need;
    return SH_OK;
}

int sh_voice_sample(sh_voice* v, const int32_t* hist, int n_frames, const double* u, float temp, float rep,
                    int32_t* picks, double* keep) {
    if (!v || n_frames < 0 || n_frames > VS_MAX_HIST || (n_frames && !hist))
        return set_error(SH_E_ARG, "sh_voice_sample: bad argument (0 <= n_frames <= 256)");
    if (v->last_need < 0) return set_error(SH_E_ARG, "sh_voice_sample: no pass has scored codebooks yet");
    const int n = v->last_need;
    if (n && (!u || !picks || !keep)) return set_error(SH_E_ARG, "sh_voice_sample: bad argument");
    if (!(temp > 0.0f) || !(rep > 0.0f)) return set_error(SH_E_ARG, "sh_voice_sample: temp and rep must be > 0");
    if (v->info.n_vocab > VS_MAX_V) return set_error(SH_E_SHAPE, "sh_voice_sample: more than 4096 codes per codebook");
    for (int j = 0; j < n; j++)
        if (!(u[j] >= 0.0 && u[j] < 1.0)) return set_error(SH_E_ARG, "sh_voice_sample: u must lie in [0, 1)");
    if (!n) return SH_OK;
    VCHK(hipSetDevice(v->device));
    sample_io& io = *v->smp_host;
    const int P = v->info.n_cb;
    for (int j = 0; j < n; j++) io.u[j] = u[j];
    memcpy(io.hist, hist, (size_t)n_frames * P * sizeof(int32_t));
    const size_t in_bytes = offsetof(sample_io, hist) + (size_t)n_frames * P * sizeof(int32_t);
    VCHK(hipMemcpyAsync(v->smp_dev, &io, in_bytes, hipMemcpyHostToDevice, v->stream));
    vsample_args a{};
    a.scores = v->out; a.V = v->info.n_vocab; a.n_cb = P;
    a.need = v->in_dev->need; a.n_need = &v->in_dev->n_need;
    a.hist = v->smp_dev->hist; a.n_frames = n_frames;
    a.u = v->smp_dev->u; a.temp = temp; a.rep = rep;
    a.picks = v->smp_dev->picks; a.keep = v->smp_dev->keep;
    VCHK(launch_vsample(a, n, v->stream));
    VCHK(hipMemcpyAsync(&io.keep, &v->smp_dev->keep, offsetof(sample_io, hist) - offsetof(sample_io, keep),
                        hipMemcpyDeviceToHost, v->stream));
    VCHK(hipStreamSynchronize(v->stream));
    for (int j = 0; j < n; j++) {
        picks[j] = io.picks[j];
        keep[j] = io.keep[j];
    }
    v->last_need = -1;   // the score rows now hold penalised scores: a pass is sampled once
    return SH_OK;
}

int sh_voice_feedback(sh_voice* v, const int32_t* codes, float* out) {
    if (!v || !codes || !out) return set_error(SH_E_ARG, "sh_voice_feedback: bad argument");
    const int P = v->info.n_cb;
    for (int i = 0; i < P; i++)
        if (codes[i] < 0 || codes[i] >= v->info.n_vocab) return set_error(SH_E_ARG, "sh_voice_feedback: code out of range");
    VCHK(hipSetDevice(v->device));
    pass_in& in = *v->in_host;
    for (int i = 0; i < VX_MAX_P; i++) in.codes[i] = i < P ? codes[i] : 0;
    in.n_need = 0;
    v->last_need = -1;   // the device copy of the pass's need list is overwritten: nothing left to sample
    VCHK(hipMemcpyAsync(v->in_dev, &in, sizeof(pass_in), hipMemcpyHostToDevice, v->stream));
    vfeed_args a{v->feed_rows, v->feed_row_bytes, v->info.n_in, v->info.n_vocab, P, v->in_dev->codes, v->fb};
    VCHK(launch_vfeed(a, v->stream));
    VCHK(hipMemcpyAsync(out, v->fb, (size_t)v->info.n_in * 4, hipMemcpyDeviceToHost, v->stream));
    VCHK(hipStreamSynchronize(v->stream));
    return SH_OK;
}

}  // extern "C"
