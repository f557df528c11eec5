// The Q8_0 voice generator on the device (imi/core/voice.{h,cpp}): table layout, kernel arguments, launchers.
//
// Arithmetic follows imi_q8g_group (imi/core/tables.cpp:324-402) per output, so every score is the number the
// CPU path computes: weights are int8 codes times an fp16 scale per 32 columns, multiplied with unrounded fp32
// inputs for the P codebook positions of a pass, in one of three fixed operation orders chosen by P:
//   generic (P not in {1, 6, 12}): per row, block and position s = sum over the 32 columns of fma(w, x, s) in column
//            order, then acc = fma(d, s, acc) over the blocks in order;
//   scaled  (P in {6, 12}):        per row and position one chain over all columns of fma(w * d, x, acc);
//   single  (one input vector):    four chains over columns k % 4 of fma(w, d * x, a), then (a0 + a1) + (a2 + a3).
#pragma once
#include <hip/hip_runtime.h>

#include <cstdint>
#include <vector>

namespace sh {

constexpr int VX_MAX_P = 12;      // codebook positions of a pass (imi/core/voice.cpp:157 keeps 12 per thread)
constexpr int VX_MAX_D = 64;      // head width the attention kernel takes (same limit, voice.cpp:157)
constexpr int VX_THREADS = 256;

// One Q8_0 table in the device layout: codes [rows_pad/8][nb][8][32] int8 (per group of 8 rows and 32-column
// block, the 8 rows' codes side by side), scales [rows_pad/8][nb][8] fp16. Rows past `rows` are zero.
struct q8dev {
    const int8_t* codes = nullptr;
    const uint16_t* scales = nullptr;
    int rows = 0, rows_pad = 0, cols = 0, nb = 0;
};

enum { VP_PLAIN = 0, VP_NORM = 1 };                        // input: as is, or rms-normed per position
enum { VE_STORE = 0, VE_RESID = 1, VE_SWIGLU = 2 };        // output: store, add into, or silu(gate) * up

// one table applied to the P positions of a pass
struct vtab_args {
    q8dev W;
    const float* src;       // input [P][src_ld]; columns [0, W.cols)
    int src_ld;
    const float* norm_w;    // VP_NORM: x * rms_scale(x) * norm_w, per position (imi/core/vec.h:36-39)
    float eps;
    float* out;             // VE_STORE: out[p][row]; VE_RESID: out[p][row] += acc; VE_SWIGLU: out[p][4 g + r]
    int out_ld;
    int units;              // workgroups: row groups per workgroup = 1 (2 for VE_SWIGLU: gate group, up group)
    float* part;            // generic order, VE_STORE/VE_RESID, nb > 32: [units][8 P][nb] scratch of per-block sums
                            // that splits the table over its 1024-column chunks (null: one workgroup per group)
};

// one table times a single input vector: the input projection (per frame) and the word scores (per pass)
struct vone_args {
    const q8dev* tabs;      // device array: scores index it by codebook; the projection passes one table
    int rows;               // output rows per table
    const float* src;       // single: input [cols]; scores: the pass's residual stream [P][E]
    const float* bias;      // added to each output (nullable)
    int head;               // 1: scores (input = head_norm(out_norm(src[cb])) for cb = need[j])
    const float* out_norm;
    const float* head_norm; // [n_cb][E]
    const int32_t* need;    // device [n_need]
    const int32_t* n_need;  // device scalar
    float eps;
    float* out;             // [j][rows]
    int rows_per_wg;        // 64
};

struct vattn_args {
    const float* qkv;       // [P][n_qkv]: q (H*D) | k (Hk*D) | v (Hk*D) | gate (H)
    int n_qkv;
    float* att;             // [P][H*D]
    const float* q_norm;
    const float* k_norm;
    const float2* rope_cs;  // [P][D/2] (cos, sin) of position p, pair i
    int P, n_head, n_kv, D;
    float eps, scale;       // scale = 1 / sqrtf(D)
};

struct vembed_args {
    const q8dev* tabs;      // device [n_cb]: codebook cb's code table (its rows are the input embeddings too)
    int E, P;
    const int32_t* codes;   // device [P]; < 0 selects mask_embd
    const float* mask;
    const float* base;      // [P][E]
    float* x;               // [P][E]
};

struct vfeed_args {
    const uint8_t* rows;    // Q8_0 rows as stored in the file: n_in / 32 blocks of (fp16 d, 32 int8)
    long long row_bytes;
    int n_in, n_vocab, n_cb;
    const int32_t* codes;   // device [n_cb]
    float* out;             // [n_in]
};

constexpr int VS_MAX_HIST = 256;   // history frames the repeat penalty may look back over
constexpr int VS_MAX_V = 4096;     // codes per codebook the sampler takes (its row lives in LDS)

// temperature sampling with a repeat penalty of one pass's scored codebooks (imi/core/talk.cpp:147-164)
struct vsample_args {
    float* scores;          // [n_need][V] the pass's scores; the penalised rows are written back
    int V, n_cb;
    const int32_t* need;    // device [n_need]: codebook of score row j
    const int32_t* n_need;  // device scalar
    const int32_t* hist;    // device [n_frames][n_cb] codes of the previous frames, oldest first
    int n_frames;
    const double* u;        // device [n_need] uniform draws in [0, 1)
    float temp, rep;
    int32_t* picks;         // device [n_need]
    double* keep;           // device [n_need] 1 - p[V - 1] / sum
};

// Q8_0 rows (each n_cols / 32 blocks of fp16 d + 32 int8) -> the device layout's codes and scales (host side)
void repack_q8(const std::vector<const uint8_t*>& rows, int cols, std::vector<int8_t>& codes, std::vector<uint16_t>& scales);

hipError_t launch_vtab(int P, int pro, int epi, const vtab_args& a, hipStream_t s);
hipError_t launch_vsample(const vsample_args& a, int max_need, hipStream_t s);
hipError_t launch_vone(const vone_args& a, int n_sets, int cols, hipStream_t s);
hipError_t launch_vattn(const vattn_args& a, hipStream_t s);
hipError_t launch_vembed(const vembed_args& a, hipStream_t s);
hipError_t launch_vfeed(const vfeed_args& a, hipStream_t s);

}  // namespace sh
