// Kernel argument blocks and launch helpers of libseoul_hip (host + device).
#pragma once
#include <hip/hip_runtime.h>
#include <cstdint>

namespace sh {

// Per-step parameters, in device memory. The host writes token/pos/state pointers before a step; the step's last
// kernel advances pos, and in a device-side greedy loop writes the chosen id back into token.
struct step_params {
    int32_t token[2];
    int32_t pos[2];
    int32_t best[2];        // argmax of the step's logits (-1 when no logits were computed)
    int32_t n_done;         // steps finished in a device-side loop
    int32_t greedy;         // 1: the next step's token is this step's argmax
    uint16_t* kc[2];        // conversation m's key cache [n_attn][n_kv][n_ctx][D] fp16
    uint16_t* vc[2];        // value cache, same layout
    float* conv[2];         // conversation m's conv memory [n_conv][d_conv][E], oldest tap first
    int32_t* out_tok[2];    // ids chosen in a device-side loop, or null
};

enum { PRO_CUT = 0, PRO_CUT_HALF_AWAY = 1, PRO_EMBED_NORM = 2, PRO_RESID_NORM = 3, PRO_PRECUT = 4 };
enum { EPI_STORE = 0, EPI_SWIGLU = 1, EPI_CONV = 2, EPI_LOGITS = 3 };

// one Q4_0 table in the device layout: codes [rows][nb][16 B] (the file's nibble bytes, scales split off),
// scales [rows/8][nb][8] fp16 (the 8 rows of a group side by side per block)
struct q4dev {
    const void* codes = nullptr;
    const void* scales = nullptr;
    const void* mins = nullptr;    // Q4_1 tables: fp16 block minima, laid out as scales; null for Q4_0
    int rows = 0, cols = 0, nb = 0;
};

// Q6_K word table (imi/core/tables.cpp:63, 215-287), 210-byte blocks of 256 values, one unit = (row, block).
// Codes: units in tiles of 64; tile t holds 13 16-byte words per unit, word-major: word w of unit u at
// [(u / 64) * 13 + w][u % 64] (words 0-7 ql, 8-11 qh, 12 the 16 int8 scales), so a wave reading one word of 64
// consecutive units reads 1 KB contiguously. d: fp16 per unit. Units past rows * nbk are zero.
struct q6dev {
    const void* codes = nullptr;
    const uint16_t* d = nullptr;
    int rows = 0, cols = 0, nbk = 0;   // nbk = cols / 256 blocks per row
};

struct gemv_args {
    q4dev W;
    int units;                 // rows / (8 * groups per unit)
    // prologue
    const float* src;          // PRO_CUT*: float input [M][src_ld]
    int src_ld;
    const float* x_in;         // residual stream [M][E]
    float* x_out;              // updated residual stream (block 0 writes it)
    const float* y_in;         // table output added after its post-norm (PRO_RESID_NORM), null = none
    const float* w_post;
    const float* w_pre;        // norm weight in front of this table
    const float* embd;         // PRO_EMBED_NORM: input vectors [M][E] used when token < 0
    q4dev emb;                 // word table (input rows)
    q6dev emb6;                // the word table when it is Q6_K (then emb is empty)
    float* hidden_out;         // if set, block 0 writes the normed input h here ([M][E])
    float eps;
    // epilogue
    float* out;                // [M][out_ld]
    int out_ld;
    const float* conv_w;       // EPI_CONV: [d_conv + 1][E]
    int conv_layer, d_conv, E;
    float* part_v;             // EPI_LOGITS: per-block best value [M][gridDim.x]
    int* part_i;               // and its row
    step_params* P;
    int upw;                   // k_gemv_norm: units per workgroup (chunk), 0 = pick
    q6dev W6;                  // k_scores_q6k: the Q6_K word table
    // EPI_SWIGLU with outq set: the SwiGLU output also cut to int8 per 32 channels (imi_cut32) by the workgroup that
    // forms them (4 units per chunk: a chunk's 32 channels are one cut block): codes [M][out_ld], d and s = d * sum
    // of the codes [M][out_ld / 32]
    int8_t* outq;
    float* outd;
    float* outs;
    // PRO_PRECUT: the input arrives cut (codes [M][src_ld], d and s [M][src_ld / 32]), as such an epilogue wrote it
    const int8_t* src_q;
    const float* src_d;
    const float* src_s;
};

// several kernel-level Q4_0 GEMVs in one launch: table t's 8-row groups are workgroups
// start[t] .. start[t + 1] - 1 (start[0] = 0, start[t + 1] - start[t] = W[t].rows / 8); src[t] [M][cols], out[t] [M][rows]
constexpr int GEMV_GROUP_MAX = 8;
struct gemv_group_args {
    int n;
    int start[GEMV_GROUP_MAX + 1];
    q4dev W[GEMV_GROUP_MAX];
    const float* src[GEMV_GROUP_MAX];
    float* out[GEMV_GROUP_MAX];
};

struct attn_args {
    const float* qkv;          // [M][ld_qkv]: q (H*D) | k (Hk*D) | v (Hk*D) | gate (H)
    int ld_qkv;
    float* att;                // [M][H*D]
    const float* q_norm;
    const float* k_norm;
    const float2* rope_cs;     // [n_ctx][D/2] (cos, sin) for this layer's base, computed on the host
    int layer_ai;              // attention layer index into the caches
    int n_head, n_kv, D, n_ctx, n_swa;
    float eps;
    step_params* P;
};

struct final_args {
    const float* x_in;         // residual stream [M][E]
    const float* y_in;         // last table output (post-norm residual), null = none
    const float* w_post;
    const float* w_out;        // output norm
    float* hidden_out;         // [M][E]
    int E;
    float eps;
    const float* part_v;       // argmax partials (null when no logits were computed)
    const int* part_i;
    int n_part;
    const float* logits;       // the word scores [M][ld_logits] the partials were taken over (row 0 is read)
    int ld_logits;
    step_params* P;
    int advance;               // 1: pos += 1 (and greedy bookkeeping)
};

}  // namespace sh
