// Internal host-side types of libseoul_hip shared by its host files (sh_engine.cpp, sh_prefill_host.cpp): the
// context, conversation states, device layers, and the kernel launchers they call. Not part of the C ABI.
#pragma once
#include <hip/hip_runtime.h>

#include <cstdint>
#include <string>
#include <vector>

#include "../../include/seoul_hip.h"
#include "sh_kernels.h"

namespace sh {
int set_error(int code, const std::string& msg);   // sets the thread's last error; returns code
int run_prefill(sh_ctx* c, sh_state* st, const int32_t* tokens, const float* embd, int n, bool want_logits,
                float* hidden_last, float* logits, float* hidden_all, int32_t* best);

hipError_t launch_gemv(int M, int pro, int epi, int grid, const gemv_args& a, hipStream_t s, hipEvent_t t0 = nullptr, hipEvent_t t1 = nullptr);
hipError_t launch_gemv_group(int M, bool half, const gemv_group_args& g, hipStream_t s, hipEvent_t t0 = nullptr, hipEvent_t t1 = nullptr);
// workgroups of a word-score launch (the argmax partials k_final reduces), at most max_grid
int gemv_logits_grid(int M, int pro, const gemv_args& a, int max_grid);
hipError_t launch_attn(int M, const attn_args& a, hipStream_t s);
// whether the FFN gate|up launch can publish its SwiGLU output cut to int8 for the down launch (PRO_PRECUT)
bool swiglu_cut_takes(int M, const gemv_args& gate_up, const gemv_args& down);
// word scores over a Q6_K table (a.W6): prologue from x_in/y_in/w_post/w_pre (or src, already normed), logits to
// a.out when set, per-workgroup first maxima to part_v / part_i [M][grid]
constexpr int SH_Q6K_GRID = 256;   // k_scores_q6k workgroups: one per compute unit, each looping over tiles
hipError_t launch_scores_q6k(int M, int grid, const gemv_args& a, hipStream_t s, hipEvent_t t0 = nullptr, hipEvent_t t1 = nullptr);
hipError_t launch_final(int M, const final_args& a, hipStream_t s);
hipError_t launch_q4_rows(const q4dev& T, const int32_t* ids, int n, float* out, hipStream_t s);
hipError_t launch_expf(const float* x, float* y, long long n, hipStream_t s);
// the longest contexts the decode and prefill attention kernels hold (their score rows live in LDS)
int attn_max_ctx(int grp, int D);
// the no-allocation product's per-device scratch address (sh_noalloc.hip), looked up once per device
int noalloc_setup(int device);
int pf_attn_max_ctx(int grp, int D);
}

namespace sh {
// one device allocation carved into 256-byte aligned pieces
struct arena {
    char* base = nullptr;
    size_t size = 0, used = 0;
    void* take(size_t n) {
        const size_t at = (used + 255) / 256 * 256;
        if (at + n > size) return nullptr;
        used = at + n;
        return base + at;
    }
};

struct layer_dev {
    bool conv = false, swa = false;
    int ai = -1, ci = -1;
    q4dev in_proj, out_proj, qkvg, o, gate_up, down;
    const float *attn_norm = nullptr, *post_attn_norm = nullptr, *ffn_norm = nullptr, *post_ffn_norm = nullptr;
    const float *q_norm = nullptr, *k_norm = nullptr, *conv_w = nullptr;
};

}  // namespace sh

using sh::arena;
using sh::layer_dev;
using sh::q4dev;
using sh::q6dev;
using sh::step_params;

struct sh_q4 {
    sh_ctx* ctx = nullptr;
    q4dev t;
    void* mem = nullptr;
};

struct sh_state {
    sh_ctx* ctx = nullptr;
    uint16_t* kc = nullptr;
    uint16_t* vc = nullptr;
    float* conv = nullptr;
    int pos = 0;
};

struct sh_ctx {
    int device = 0;
    hipStream_t stream = nullptr;
    hipEvent_t ev0 = nullptr, ev1 = nullptr;
    bool loaded = false;
    sh_model_info info{};
    float eps = 1e-5f, rope_base = 1e6f, rope_base_swa = 1e4f;
    arena w;                         // weights + norms + rope tables
    std::vector<layer_dev> layers;
    q4dev vocab;                     // tied word table when it is Q4_0
    q6dev vocab6;                    // tied word table when it is Q6_K (imi's own format)
    const float* out_norm = nullptr;
    const float2* rope_cs = nullptr;
    const float2* rope_cs_swa = nullptr;
    int n_conv = 0, nqkv = 0;
    // work buffers (device)
    arena work;
    float *xbuf[2] = {nullptr, nullptr}, *y = nullptr, *u = nullptr, *qkv = nullptr, *att = nullptr, *act = nullptr, *fo = nullptr;
    float *hidden = nullptr, *logits = nullptr, *embd_stage = nullptr, *part_v = nullptr;
    int8_t* act_q = nullptr;          // the FFN activation cut to int8 per 32 channels [2][n_ff], with d and s [2][n_ff / 32]
    float *act_d = nullptr, *act_s = nullptr;
    int* part_i = nullptr;
    int32_t* gen_out = nullptr;       // device-side greedy ids [2][gen_cap]
    int gen_cap = 0;
    float* bench_x = nullptr;         // kernel-API input/output staging
    float* bench_y = nullptr;
    size_t bench_cap = 0;
    step_params* P_dev = nullptr;
    step_params* P_host = nullptr;    // pinned
    int vocab_grid = 2048;
    hipGraphExec_t graph[3][2] = {{nullptr, nullptr}, {nullptr, nullptr}, {nullptr, nullptr}};
    std::vector<sh_state*> states;    // live children: destroying the context releases their device memory
    std::vector<sh_q4*> tables;
    // the step replays a captured graph; SEOUL_HIP_GRAPHS=0 enqueues the same kernels directly (for tools that do
    // not trace graph launches)
    bool use_graphs = true;
    // prefill work buffers (PF_MAX_N positions, made on first use)
    char* pf_mem = nullptr;
    float *pf_x = nullptr, *pf_y = nullptr, *pf_big = nullptr, *pf_act = nullptr, *pf_hid = nullptr;
    int8_t* pf_q = nullptr;
    float *pf_d = nullptr, *pf_s = nullptr, *pf_emb = nullptr;
    int32_t* pf_tok = nullptr;
    bool use_prefill = true;          // SEOUL_HIP_PREFILL=0: step_batch runs n single steps instead
    // the FFN gate|up launch cuts its output for the down launch (SEOUL_HIP_PRECUT=0: down cuts the floats itself)
    bool use_precut = true;
    // set while sh_bench_step_kernel runs steps without the graph: one kind of the step's GEMV launches (0 FFN
    // gate|up, 1 FFN down, 2 Q4_0 word scores) records this event pair list around each kernel
    std::vector<hipEvent_t>* probe_ev = nullptr;
    int probe_kind = -1, probe_used = 0;
};

