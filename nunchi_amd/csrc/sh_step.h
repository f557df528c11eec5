// The persistent step kernel's program and parameters (host + device).
//
// A decode step is a fixed sequence of stages (per layer: the first table read, then the conv or attention part,
// then FFN gate|up and down; at the end the word scores or the final norm). One cooperative launch runs n steps of
// it on every compute unit at once. Stage outputs travel as tagged 8-byte records (32-bit value, 32-bit step
// epoch), so a consumer's wait on the data itself is the only synchronisation between stages; each workgroup
// prefetches the weights of its next chunk of work before it waits.
#pragma once
#include <hip/hip_runtime.h>

#include <cstdint>

#include "sh_kernels.h"

namespace sh {

enum { SK_GEMV = 0, SK_ATTN = 1, SK_VOCAB = 2 };
enum { SKP_FIRST = 0, SKP_RESID = 1, SKP_CUT = 2 };
enum { SKE_STORE = 0, SKE_SWIGLU = 1, SKE_CONV = 2, SKE_LOGITS = 3 };

constexpr int SK_THREADS = 512;
constexpr int SK_CONV_MAX = 7;                     // conv memory taps (d_conv) the kernel takes

// LDS map of the step kernel (bytes)
// x and y hold E <= 2048 values per conversation transposed: value i at (i % 32) * SK_XT_LD + i / 32, so lane P of
// a norm's AVX2-order chain (the squares of values P, P + 32, P + 64, ...) reads its operands 4 at a time
constexpr int SK_XT_LD = 68;                       // row stride (floats): 64 + 4 keeps 16-byte reads conflict free
constexpr int SK_XT_M = 32 * SK_XT_LD;             // floats per conversation
constexpr int SK_OFF_X = 0;                        // float [2][32][68] residual stream, private to the workgroup
constexpr int SK_OFF_Y = SK_OFF_X + 8 * SK_XT_M;   // float [2][32][68] table output feeding a norm
constexpr int SK_OFF_XQ = SK_OFF_Y + 8 * SK_XT_M;  // int8 [2][8192] the cut input
constexpr int SK_OFF_DX = SK_OFF_XQ + 16384;       // float [2][256] cut scales
constexpr int SK_OFF_S = SK_OFF_DX + 2048;         // float [2][256] d * sum(q) per block
constexpr int SK_OFF_OPS = SK_OFF_S + 2048;        // float2 [nb][C + 1] chain operands / input staging / attention
constexpr int SK_OPS_BYTES = 70656;
constexpr int SK_OFF_DD = SK_OFF_OPS + SK_OPS_BYTES;   // float [nb][rows + 1] weight scales
constexpr int SK_DD_BYTES = 18432;
constexpr int SK_OFF_COR = SK_OFF_DD + SK_DD_BYTES;    // float [256]
constexpr int SK_OFF_OUT = SK_OFF_COR + 1024;          // float [256]
constexpr int SK_OFF_RED = SK_OFF_OUT + 1024;          // float [512] + int [512]
constexpr int SK_OFF_MISC = SK_OFF_RED + 4096;         // small scalars
constexpr int SK_OFF_RNG = SK_OFF_MISC + 256;          // int4 [SK_MAX_STAGES] this workgroup's unit range per stage
constexpr int SK_MAX_STAGES = 128;
constexpr int SK_OFF_CL = SK_OFF_RNG + 16 * SK_MAX_STAGES;   // int [SK_MAX_CHUNKS + 1] this workgroup's chunks of a step
constexpr int SK_MAX_CHUNKS = 511;
constexpr int SK_LDS_BYTES = SK_OFF_CL + 4 * (SK_MAX_CHUNKS + 1);
constexpr int SK_ATTN_BYTES = SK_OPS_BYTES + SK_DD_BYTES;   // attention's share (OPS and DD are contiguous)

// groups of 8 rows per chunk for a table of nb 32-column blocks and M inputs: one (group, block) pair per thread in
// phase 1, and per row the chain operands float(isum) and d * dx ([2][M][rows][st]) and the scales d ([rows][st])
// in LDS, st the row stride below
__host__ __device__ inline int sk_row_stride(int nb) { return ((nb + 3) & ~3) + 4; }   // 16-byte rows, odd in 16 B
__host__ __device__ inline int sk_gmax(int nb, int M) {
    const int st = 4 * sk_row_stride(nb);   // bytes per row of one block-ordered array
    int g = SK_THREADS / nb;
    const int c1 = 256 / (8 * M);   // chains (input, row) per chunk <= 256: the epilogue's exchange buffer
    const int c2 = (SK_DD_BYTES - 64) / (8 * st);
    const int c3 = (SK_OPS_BYTES - 64) / (8 * 2 * M * st);   // 64 B left for the chain's read-ahead
    g = g < c1 ? g : c1;
    g = g < c2 ? g : c2;
    g = g < c3 ? g : c3;
    return g;
}

struct sk_stage {
    int kind, pro, epi;
    q4dev W;
    int ug;                           // groups of 8 rows per unit: 1, 2 (gate|up), 3 (conv b|c|x)
    int units;                        // W.rows / (8 * ug)
    const unsigned long long* in;     // input records [2 parity][2 conversations][n_in]
    int n_in;
    unsigned long long* out;          // output records [2][2][n_out]
    int n_out;
    const float* w_post;              // SKP_RESID: x += norm(y) * w_post
    const float* w_pre;               // h = norm(x) * w_pre
    const float* conv_w;              // SKE_CONV: taps [d_conv + 1][E]
    int conv_layer;
    int cut_out;                      // SKE_SWIGLU: publish the output already cut, per 32 values 10 records
                                      // (8 words of int8 codes, d, d * sum) instead of 32 floats
    int cut_in;                       // SKP_CUT: the input comes in that form
    int layer_ai, swa;                // SK_ATTN
    const float* q_norm;
    const float* k_norm;
    const float2* rope_cs;
};

struct sk_conv {                      // one conversation of a launch
    uint16_t* kc;                     // key cache [n_attn][n_kv][n_ctx][D] fp16
    uint16_t* vc;
    float* conv;                      // conv memory [n_conv][d_conv][E]
    int pos;                          // position of step 0
    int first_token;                  // greedy launches: token of step 0 (< 0: embd row 0)
    const int32_t* tokens;            // [n_steps] device, or null for greedy; < 0 selects the embd row
    const float* embd;                // [n_steps][E] device rows for tokens < 0
    int32_t* ids;                     // [n_steps] first index of the maximum word score of each step (nullable)
    float* hidden;                    // hidden state out: row per step (hidden_stride = E) or the last step's
    int hidden_stride;
    float* logits;                    // [V] word scores of the steps that compute them (nullable)
};

struct sk_params {
    const sk_stage* stages;
    int n_stages;
    int E, n_head, n_kv, D, n_ctx, n_swa, d_conv, V;
    float eps;
    q4dev vocab;                      // tied word table (input rows)
    int n_steps, logits_from, greedy;
    unsigned epoch0;                  // tag of step 0; step i writes tag epoch0 + i into buffer parity (tag & 1)
    sk_conv cv[2];
    unsigned long long* part;         // argmax partials [2 parity][2 conversations][2 value|index][G]
    int* err;                         // set to 1 when a wait passes `timeout` wall-clock ticks
    long long timeout;
    long long* trace;                 // optional per-workgroup stage timestamps [G][n_trace]
    int n_trace;
};

hipError_t launch_step_kernel(int M, const sk_params& p, int grid, hipStream_t s);
hipError_t step_kernel_occupancy(int M, int* blocks_per_cu);

}  // namespace sh
