// The prefill ("hearing window", imi_seoul::step_batch, imi/core/seoul.cpp:490-655) on the device: argument blocks
// and launchers of its kernels. n positions go through every table at once: the table reads are int8 matrix-core
// products (v_mfma_i32_16x16x32_i8, one 32-column block per product, so each block's integer sum is exact) followed
// by imi's per-row fp32 chains over the blocks, which makes every output the number n single steps would give.
#pragma once
#include <hip/hip_runtime.h>

#include <cstdint>

#include "sh_kernels.h"

namespace sh {

constexpr int PF_MAX_N = 512;   // positions per device chunk (larger batches run in chunks; results do not change)

// n input rows cut to int8 per 32 columns, block-major (imi_q8b, imi/core/tables.cpp:405-416)
struct pf_cut {
    int8_t* q = nullptr;    // [nb][n][32]
    float* d = nullptr;     // [nb][n] scale amax / 127
    float* s = nullptr;     // [nb][n] d * sum(q)
};

enum { PFR_FIRST = 0, PFR_RESID = 1 };

struct pf_conv_args {       // gated short conv along positions, then the cut of its output
    const float* bcx;       // [n][3E] in_proj output: per 8 channels, 8 b rows, 8 c rows, 8 x rows
    const float* w;         // [d_conv + 1][E] taps, the newest last
    float* state;           // [d_conv][E] this layer's conv memory, oldest tap first
    int n, E, d_conv;
    pf_cut cut;
};

// one workgroup per position: the layer's first norm (after the embedding) or the post-norm residual, then the
// norm in front of the next table and its cut (or the output norm into hidden rows)
struct pf_rows_args {
    int n, E;
    float eps;
    const int32_t* tokens;  // PFR_FIRST: [n] device, or null (every row from embd)
    const float* embd;      // PFR_FIRST: [n][E] rows of positions whose token < 0
    q4dev vocab;            // PFR_FIRST: the tied word table (input rows)
    q6dev vocab6;           // PFR_FIRST: the word table when it is Q6_K (then vocab is empty)
    float* x;               // [n][E] residual stream (written by PFR_FIRST, updated by PFR_RESID)
    const float* y;         // PFR_RESID: [n][E] the table output the post-norm applies to
    const float* w_post;
    const float* w_pre;     // h = norm(x) * w_pre
    pf_cut cut;             // cut of h (q null: none)
    float* hidden;          // [n][E] h rows (null: none)
    pf_conv_args conv;      // PFR_RESID with conv.state set: a conv layer's memory update (the last d_conv positions'
                            // b x values) done by extra workgroups of this launch, after the conv has read the memory
};

struct pf_gemm_args {
    q4dev W;
    int n;
    pf_cut in;              // the input, cut (W.nb blocks)
    float* out;             // EPI_STORE: [n][out_ld] rows of W; EPI_SWIGLU: [n][out_ld] silu(gate) * up channels
    int out_ld;
    pf_cut outc;            // EPI_SWIGLU with outc.q set: the channels cut (out_ld / 32 blocks) instead of stored
};

struct pf_cutk_args {       // cut of n rows of K floats
    const float* src;
    int ld, K, n;
    pf_cut cut;
};


struct pf_attn_args {       // causal attention of n positions (keys and values of all of them in the cache first)
    const float* qkv;       // [n][ld]: q (H*D) | k (Hk*D) | v (Hk*D) | gate (H)
    int ld;
    const float* q_norm;
    const float* k_norm;
    const float2* rope_cs;  // [n_ctx][D/2] (cos, sin) of this layer's rope base
    uint16_t* kc;           // this layer's caches [n_kv][n_ctx][D] fp16
    uint16_t* vc;
    int n, pos0, n_head, n_kv, D, n_ctx, n_swa;
    float eps;
    pf_cut cut;             // cut of the attention output rows [n][H*D]
};

hipError_t launch_pf_rows(int mode, const pf_rows_args& a, hipStream_t s);
hipError_t launch_pf_gemm(int epi, const pf_gemm_args& a, hipStream_t s);
// whether launch_pf_gemm takes EPI_SWIGLU with the cut output for these arguments (the staged kernel, whole 64-row
// workgroups, each one 32-channel block)
bool pf_swiglu_cut_takes(const pf_gemm_args& a);
hipError_t launch_pf_cut(const pf_cutk_args& a, hipStream_t s);
// the conv along positions and its cut; the conv memory update rides on the next launch_pf_rows (its conv field)
hipError_t launch_pf_conv_lanes(const pf_conv_args& a, hipStream_t s);
hipError_t launch_pf_kv(const pf_attn_args& a, hipStream_t s);
hipError_t launch_pf_attn(const pf_attn_args& a, hipStream_t s);

}  // namespace sh
