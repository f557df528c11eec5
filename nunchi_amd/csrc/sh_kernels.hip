// HIP kernels of the brain step (gfx950, wave64): the Q4_0 GEMV family with fused prologues (embedding, post-norm
// residual, RMS norm, int8 input cut) and epilogues (store, SwiGLU, short conv, word scores), GQA decode attention,
// and the step's final norm / argmax.
//
// Arithmetic follows imi's engine (imi/core/seoul.cpp:359-488, imi/core/tables.cpp:100-198, imi/core/vec.h): the
// input of every table is cut to int8 per 32 values, each 32-column block's integer dot is exact, and the fp32
// epilogue per block is  float(isum) * (d * dx) - d * (8 * dx * sum(xq))  summed over blocks.
#include <hip/hip_ext.h>

#include "sh_device.h"
#include "sh_kernels.h"

#include <algorithm>
#include <cstddef>

namespace sh {

// ---------------------------------------------------------------- helpers
__device__ __forceinline__ void load32(const float* p, float* v) {
    const f32x4* q = (const f32x4*)p;
#pragma unroll
    for (int k = 0; k < 8; k++) { const f32x4 t = q[k]; v[4 * k] = t.x; v[4 * k + 1] = t.y; v[4 * k + 2] = t.z; v[4 * k + 3] = t.w; }
}
__device__ __forceinline__ void store32(float* p, const float* v) {
    f32x4* q = (f32x4*)p;
#pragma unroll
    for (int k = 0; k < 8; k++) q[k] = f32x4{v[4 * k], v[4 * k + 1], v[4 * k + 2], v[4 * k + 3]};
}

// Q4_0 row block (device layout) -> 32 floats (code - 8) * d
__device__ __forceinline__ void q4_dequant_block(const q4dev& T, int row, int blk, float* v) {
    const u32x4 c = ((const u32x4*)T.codes)[(size_t)row * T.nb + blk];
    const uint16_t dh = ((const uint16_t*)T.scales)[((size_t)(row >> 3) * T.nb + blk) * 8 + (row & 7)];
    const float d = h2f(dh);
    const unsigned w[4] = {c.x, c.y, c.z, c.w};
#pragma unroll
    for (int i = 0; i < 16; i++) {
        const unsigned byte = (w[i >> 2] >> (8 * (i & 3))) & 0xFFu;
        v[i] = (float)((int)(byte & 15u) - 8) * d;
        v[16 + i] = (float)((int)(byte >> 4) - 8) * d;
    }
}

// half r (0..7) of a 16-byte word of 8 fp16 values, as float
__device__ __forceinline__ float half_of(const u32x4& w, int r) {
    const unsigned word = (r >> 1) == 0 ? w.x : (r >> 1) == 1 ? w.y : (r >> 1) == 2 ? w.z : w.w;
    return h2f((uint16_t)((r & 1) ? (word >> 16) : (word & 0xFFFFu)));
}

// ---------------------------------------------------------------- Q4_0 GEMV
// One wave per block; a unit is UG groups of 8 rows (R rows).
// Phase 1, lanes over input blocks: lane j owns blocks j, j + 64, ... (< nb); it cuts them itself (int8 codes stay in
// registers) and, per row, loads its 16 B of codes (one row = 1 KB per load for the wave) and the 8 rows' scales of
// the block (16 B), and computes each (row, block) integer dot exactly. The dots and scales go to LDS.
// Phase 2, lanes over rows: lane (m, k) runs imi's per-row chain over blocks j in order
// (imi/core/tables.cpp:127-143): acc = fma(float(isum), d * dx, acc), cor = fma(d, s, cor), out = acc - 8 cor
// (q4x8, imi/kernels/q4x8.cpp:51-77: cor = fma(d, corr, cor), out = acc - cor) -- the same fp32 operations in the
// same order as the CPU, so the outputs are the CPU's bit for bit.
template <int PRO> constexpr bool norm_staging() { return PRO == PRO_EMBED_NORM || PRO == PRO_RESID_NORM; }

template <int M, int NBL, int PRO, int EPI, int UG>
__global__ __launch_bounds__(64) void k_gemv(gemv_args a) {
    constexpr int R = 8 * UG;
    constexpr int LDI = M * R + 1;   // odd strides: phase-1 writes (lanes over blocks) and phase-2 reads (lanes
    constexpr int LDD = R + 1;       // over rows) are both free of LDS bank conflicts
    extern __shared__ float lds[];
    const int lane = threadIdx.x;
    const int nb = a.W.nb;
    int* l_isum = (int*)lds;                       // [nb][LDI]
    float* l_d = lds + (size_t)nb * LDI;           // [nb][LDD]
    float* l_dx = l_d + (size_t)nb * LDD;          // [M][nb]
    float* l_s = l_dx + (size_t)M * nb;            // [M][nb]
    float* l_x = l_s + (size_t)M * nb;             // [E] staging for the norms
    float* l_m = l_x + (norm_staging<PRO>() ? a.E : 0);   // [nb][LDD] Q4_1 block minima (a.W.mins set)
    const bool hm = a.W.mins != nullptr;
    int xq[M][NBL][8];

    // ---- prologue: the input of this table, cut to int8 per 32 ----
    if (PRO == PRO_CUT || PRO == PRO_CUT_HALF_AWAY) {
#pragma unroll
        for (int m = 0; m < M; m++)
#pragma unroll
            for (int b = 0; b < NBL; b++) {
                const int blk = lane + 64 * b;
#pragma unroll
                for (int w = 0; w < 8; w++) xq[m][b][w] = 0;
                if (blk < nb) {
                    float v[32];
                    load32(a.src + (size_t)m * a.src_ld + 32 * blk, v);
                    int sum;
                    const float d = cut32(v, xq[m][b], &sum, PRO == PRO_CUT_HALF_AWAY);
                    l_dx[m * nb + blk] = d;
                    // imi_q8::from (tables.cpp:107): s = d * sum; quant_in (q4x8.cpp:46): corr = 8 * d * sum
                    l_s[m * nb + blk] = PRO == PRO_CUT ? d * (float)sum : 8.0f * d * (float)sum;
                }
            }
    } else {
        // PRO_EMBED_NORM / PRO_RESID_NORM: lane j holds columns 32j..32j+31 (nb <= 64)
        const int E = a.E;
        const bool on = lane < nb;
#pragma unroll
        for (int m = 0; m < M; m++) {
            float xv[32];
#pragma unroll
            for (int i = 0; i < 32; i++) xv[i] = 0.0f;
            if (PRO == PRO_EMBED_NORM) {
                const int tok = a.P->token[m];
                if (on) {
                    if (tok >= 0 && a.emb6.codes) q6k_dequant32((const u32x4*)a.emb6.codes, a.emb6.d, a.emb6.nbk, tok, lane, xv);
                    else if (tok >= 0) q4_dequant_block(a.emb, tok, lane, xv);
                    else load32(a.embd + (size_t)m * E + 32 * lane, xv);
                }
            } else {
                if (on) load32(a.x_in + (size_t)m * E + 32 * lane, xv);
                if (a.y_in) {   // x += norm(y) * w_post  (imi_norm_mul_add, imi/core/vec.h:41-44)
                    float yv[32], wp[32];
                    if (on) {
                        load32(a.y_in + (size_t)m * E + 32 * lane, yv);
                        load32(a.w_post + 32 * lane, wp);
                        store32(l_x + 32 * lane, yv);
                    }
                    __syncthreads();
                    const float sc = rms_scale_wave(l_x, E, a.eps);
                    __syncthreads();
                    if (on)
#pragma unroll
                        for (int i = 0; i < 32; i++) xv[i] = fmaf(yv[i] * sc, wp[i], xv[i]);
                }
            }
            if (blockIdx.x == 0 && on && a.x_out) store32(a.x_out + (size_t)m * E + 32 * lane, xv);
            // h = norm(x) * w_pre  (imi_norm_mul, imi/core/vec.h:36-39)
            if (on) store32(l_x + 32 * lane, xv);
            __syncthreads();
            const float sc = rms_scale_wave(l_x, E, a.eps);
            __syncthreads();
            float h[32];
            if (on) {
                float wv[32];
                load32(a.w_pre + 32 * lane, wv);
#pragma unroll
                for (int i = 0; i < 32; i++) h[i] = xv[i] * sc * wv[i];
            } else {
#pragma unroll
                for (int i = 0; i < 32; i++) h[i] = 0.0f;
            }
            if (a.hidden_out && blockIdx.x == 0 && on) store32(a.hidden_out + (size_t)m * E + 32 * lane, h);
            int sum;
            const float d = cut32(h, xq[m][0], &sum, false);
            if (on) {
                l_dx[m * nb + lane] = d;
                l_s[m * nb + lane] = d * (float)sum;
            }
        }
    }
    __syncthreads();

    float best_v = -INFINITY;
    int best_i = 0x7fffffff;
    const u32x4* codes = (const u32x4*)a.W.codes;
    const u32x4* scales = (const u32x4*)a.W.scales;
    for (int u = blockIdx.x; u < a.units; u += gridDim.x) {
        // ---- phase 1: exact integer dots, lanes over blocks ----
#pragma unroll
        for (int gi = 0; gi < UG; gi++) {
            const int g = u * UG + gi;
            u32x4 c[8][NBL], s8[NBL], m8[NBL];
#pragma unroll
            for (int b = 0; b < NBL; b++) {
                const int blk = lane + 64 * b;
                if (blk < nb) {
#pragma unroll
                    for (int r = 0; r < 8; r++) c[r][b] = __builtin_nontemporal_load(codes + (size_t)(8 * g + r) * nb + blk);
                    s8[b] = __builtin_nontemporal_load(scales + (size_t)g * nb + blk);
                    // (issued on every path, so the compiler's wait counts stay exact; Q4_0 re-reads the scales)
                    m8[b] = __builtin_nontemporal_load((const u32x4*)(hm ? a.W.mins : a.W.scales) + (size_t)g * nb + blk);
                }
            }
#pragma unroll
            for (int b = 0; b < NBL; b++) {
                const int blk = lane + 64 * b;
                if (blk < nb) {
#pragma unroll
                    for (int r = 0; r < 8; r++) {
                        const unsigned sw = (r < 2) ? s8[b].x : (r < 4) ? s8[b].y : (r < 6) ? s8[b].z : s8[b].w;
                        l_d[blk * LDD + gi * 8 + r] = h2f((uint16_t)((r & 1) ? (sw >> 16) : (sw & 0xFFFFu)));
                        if (hm) l_m[blk * LDD + gi * 8 + r] = half_of(m8[b], r);
#pragma unroll
                        for (int m = 0; m < M; m++) l_isum[blk * LDI + m * R + gi * 8 + r] = q4_block_dot(c[r][b], xq[m][b]);
                    }
                }
            }
        }
        __syncthreads();
        // ---- phase 2: imi's per-row fp32 chain over the blocks, lanes over (input, row) ----
        float outv = 0.0f;
        if (lane < M * R) {
            const int m = lane / R, k = lane - m * R;
            const float* dx = l_dx + m * nb;
            const float* sv = l_s + m * nb;
            float acc = 0.0f, cor = 0.0f;
#pragma unroll 8
            for (int j = 0; j < nb; j++) {
                const float d = l_d[j * LDD + k];
                acc = fmaf((float)l_isum[j * LDI + lane], d * dx[j], acc);
                cor = fmaf(hm ? l_m[j * LDD + k] : d, sv[j], cor);   // Q4_1: the block minimum
            }
            outv = PRO == PRO_CUT_HALF_AWAY ? acc - cor : hm ? acc + cor : fmaf(-8.0f, cor, acc);
        }
        __syncthreads();
        // ---- epilogue: lane (m, k) holds row k of the unit for input m ----
        const int m = lane / R, k = lane - (lane / R) * R;
        if (EPI == EPI_STORE) {
            if (lane < M * R) a.out[(size_t)m * a.out_ld + R * u + k] = outv;
        } else if (EPI == EPI_SWIGLU) {   // unit = (gate group, up group) of 8 FFN channels (imi/core/seoul.cpp:380-394)
            const float up = __shfl(outv, (lane + 8) & 63);
            if (lane < M * R && k < 8) a.out[(size_t)m * a.out_ld + 8 * u + k] = silu(outv) * up;
        } else if (EPI == EPI_CONV) {     // unit = (b, c, x) groups of 8 channels (imi/core/seoul.cpp:407-423)
            const float cc = __shfl(outv, (lane + 8) & 63), xx = __shfl(outv, (lane + 16) & 63);
            if (lane < M * R && k < 8) {
                const int e = 8 * u + k, E = a.E, dc = a.d_conv;
                SH_GLOBAL float* st = global_ptr(a.P->conv[m]) + (size_t)a.conv_layer * dc * E;
                const float bx = outv * xx;
                float uu = outv * xx * a.conv_w[(size_t)dc * E + e];
                for (int t = 0; t < dc; t++) uu = fmaf(st[(size_t)t * E + e], a.conv_w[(size_t)t * E + e], uu);
                uu *= cc;
                for (int t = 0; t + 1 < dc; t++) st[(size_t)t * E + e] = st[(size_t)(t + 1) * E + e];
                st[(size_t)(dc - 1) * E + e] = bx;
                a.out[(size_t)m * a.out_ld + e] = uu;
            }
        } else {   // EPI_LOGITS: scores, and this lane's best (first index of the maximum)
            if (lane < M * R) {
                const int row = R * u + k;
                if (a.out) a.out[(size_t)m * a.out_ld + row] = outv;
                if (outv > best_v || (outv == best_v && row < best_i)) { best_v = outv; best_i = row; }
            }
        }
    }
    if (EPI == EPI_LOGITS) {
        // per input m: reduce over the lanes of that input
#pragma unroll
        for (int mm = 0; mm < M; mm++) {
            float v = (lane < M * R && lane / R == mm) ? best_v : -INFINITY;
            int i = (lane < M * R && lane / R == mm) ? best_i : 0x7fffffff;
#pragma unroll
            for (int o = 32; o > 0; o >>= 1) {
                const float ov = __shfl_xor(v, o);
                const int oi = __shfl_xor(i, o);
                if (ov > v || (ov == v && oi < i)) { v = ov; i = oi; }
            }
            if (lane == 0) { a.part_v[mm * gridDim.x + blockIdx.x] = v; a.part_i[mm * gridDim.x + blockIdx.x] = i; }
        }
    }
}

// ---------------------------------------------------------------- Q4_0 GEMV with the input cut (decode tables,
// kernel-level API): one 256-thread workgroup per 8-row group, NB = 64, 128 or 256 blocks per row. Every step is
// spread over the whole workgroup, so its critical path is short:
//  - loads: each thread first loads its share of the input (32 / TPB values of one block, TPB = 256 / NB threads
//    per block), then the codes of its RPT = NB / 32 rows of one block and the group's 8 scales of that block;
//  - cut (imi_cut32, imi/core/vec.h:47-75): the TPB threads of a block reduce amax and the code sum across lanes
//    (max and integer sums do not depend on order); codes, d and s to LDS; it waits only for the input loads;
//  - dots: thread (row subset, block) forms its rows' exact integer dots and writes the chain operands float(isum),
//    d * dx and d to LDS row-major;
//  - chains (imi/core/tables.cpp:127-143): wave 0, lane (m, r) acc = fma(float(isum), d * dx, acc), lane 8 M + (m, r)
//    cor = fma(d, s, cor), the same instruction stream for both (operands through per-lane row pointers), four
//    blocks per 16-byte LDS read with later reads in flight; out = fma(-8, cor, acc), or acc - cor with q4x8's
//    corr = 8 d sum (imi/kernels/q4x8.cpp:45-77).
// HM: the table is Q4_1 (imi/core/tables.cpp:127-143 with HAS_M): the correction chain takes the block minimum m in
// place of d and the row ends as acc + cor
// g: the table's 8-row group this workgroup computes
// PRE: the input arrives cut (PRO_PRECUT: codes, d and s as the FFN gate|up epilogue wrote them); the prologue only
// stages them. NR: the table has nb = a.W.nb blocks per row, a multiple of 16 below NB (an FFN of 7680 gives a 240-block
// down table): the body keeps NB's thread layout, threads past nb read the last block (their LDS slots are never
// read), strides and the chain's length follow nb
template <int M, bool HALF, int NB, bool HM, bool PRE = false, bool NR = false>
__device__ __forceinline__ void gemv_cut_body(const gemv_args& a, const int g) {
    constexpr int TPB = 256 / NB, VPT = 32 / TPB, RPT = NB / 32, ST = NB + 4, IPT = 8 / TPB;
    const int nbr = NR ? a.W.nb : NB;   // blocks per row
    extern __shared__ __align__(16) float lds[];
    int* l_xq = (int*)lds;                      // [M][NB][8] int8 codes of the cut input, 4 per word
    float* l_dx = lds + M * NB * 8;             // [M][NB]
    float* l_s = l_dx + M * NB;                 // [M][ST] s = d * sum (q4x8: 8 * d * sum)
    float* l_op = l_s + M * ST;                 // [M][8][ST] float(isum)
    float* l_oq = l_op + M * 8 * ST;            // [M][8][ST] d * dx
    float* l_dd = l_oq + M * 8 * ST;            // [8][ST] d
    const int t = threadIdx.x, lane = t & 63;
    // input share first: block jc, values part * VPT .. + VPT - 1
    const int jc = t / TPB, part = t - jc * TPB, jcl = NR ? min(jc, nbr - 1) : jc;
    f32x4 xin[PRE ? 1 : M][VPT / 4];
    u32x4 qin[PRE ? M : 1][(IPT + 3) / 4];   // PRE: this thread's IPT dwords (4 codes each) of block jc
    float din[M], sin_[M];
    if (PRE) {
        static_assert(IPT == 8 || IPT == 4 || IPT == 2, "cut dwords per thread");
#pragma unroll
        for (int m = 0; m < M; m++) {
            const unsigned* qs = (const unsigned*)(a.src_q + (size_t)m * a.src_ld + 32 * jcl) + IPT * part;
            if (IPT >= 4) {
#pragma unroll
                for (int k = 0; k < IPT / 4; k++) qin[m][k] = ((const u32x4*)qs)[k];
            } else {
                typedef unsigned u32x2 __attribute__((ext_vector_type(2)));
                const u32x2 v2 = *(const u32x2*)qs;
                qin[m][0] = u32x4{v2.x, v2.y, 0u, 0u};
            }
            din[m] = a.src_d[(size_t)m * nbr + jcl];
            sin_[m] = a.src_s[(size_t)m * nbr + jcl];
        }
    } else {
#pragma unroll
        for (int m = 0; m < M; m++) {
            const f32x4* src = (const f32x4*)(a.src + (size_t)m * a.src_ld + 32 * jcl + VPT * part);
#pragma unroll
            for (int k = 0; k < VPT / 4; k++) xin[PRE ? 0 : m][k] = src[k];
        }
    }
    // then the weights: rows sub * RPT .. + RPT - 1 of block jw
    const int jw = t % NB, sub = t / NB, jwl = NR ? min(jw, nbr - 1) : jw;
    u32x4 c[RPT];
    const u32x4* codes = (const u32x4*)a.W.codes + (size_t)(8 * g + sub * RPT) * nbr + jwl;
#pragma unroll
    for (int k = 0; k < RPT; k++) c[k] = __builtin_nontemporal_load(codes + (size_t)k * nbr);
    const u32x4 s8 = __builtin_nontemporal_load((const u32x4*)a.W.scales + (size_t)g * nbr + jwl);
    u32x4 m8 = s8;
    if (HM) m8 = __builtin_nontemporal_load((const u32x4*)a.W.mins + (size_t)g * nbr + jwl);
    // the cut of block jc by its TPB threads (PRE: staged as it arrived)
#pragma unroll
    for (int m = 0; m < M; m++) {
        if (PRE) {
#pragma unroll
            for (int w = 0; w < IPT; w++) {
                const u32x4 q4 = qin[m][w >> 2];
                l_xq[(m * NB + jc) * 8 + IPT * part + w] = (int)((w & 3) == 0 ? q4.x : (w & 3) == 1 ? q4.y : (w & 3) == 2 ? q4.z : q4.w);
            }
            if (part == 0) {
                l_dx[m * NB + jc] = din[m];
                l_s[m * ST + jc] = sin_[m];
            }
            continue;
        }
        float v[VPT];
#pragma unroll
        for (int k = 0; k < VPT / 4; k++) {
            const f32x4 xk = xin[PRE ? 0 : m][k];
            v[4 * k] = xk.x; v[4 * k + 1] = xk.y; v[4 * k + 2] = xk.z; v[4 * k + 3] = xk.w;
        }
        float amax = 0.0f;
#pragma unroll
        for (int i = 0; i < VPT; i++) amax = fmaxf(amax, fabsf(v[i]));
        if (TPB >= 2) amax = fmaxf(amax, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(amax), 0xB1, 0xF, 0xF, true)));
        if (TPB >= 4) amax = fmaxf(amax, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(amax), 0x4E, 0xF, 0xF, true)));
        const float d = amax / 127.0f;
        const float id = d != 0.0f ? 1.0f / d : 0.0f;
        int sum = 0;
#pragma unroll
        for (int w = 0; w < VPT / 4; w++) {
            unsigned packed = 0;
#pragma unroll
            for (int k = 0; k < 4; k++) {
                const float q = v[4 * w + k] * id;
                const int cq = (int)(HALF ? roundf(q) : rintf(q));
                sum += cq;
                packed |= ((unsigned)cq & 0xFFu) << (8 * k);
            }
            l_xq[(m * NB + jc) * 8 + part * (VPT / 4) + w] = (int)packed;
        }
        if (TPB >= 2) sum += __builtin_amdgcn_update_dpp(0, sum, 0xB1, 0xF, 0xF, true);
        if (TPB >= 4) sum += __builtin_amdgcn_update_dpp(0, sum, 0x4E, 0xF, 0xF, true);
        if (part == 0) {
            l_dx[m * NB + jc] = d;
            l_s[m * ST + jc] = HALF ? 8.0f * d * (float)sum : d * (float)sum;
        }
    }
    __syncthreads();
    // exact dots of rows sub * RPT .. against block jw
    {
        const unsigned sw[4] = {s8.x, s8.y, s8.z, s8.w};
        float d[RPT];
#pragma unroll
        for (int k = 0; k < RPT; k++) {
            const int r = sub * RPT + k;
            const unsigned word = RPT == 8 ? sw[k >> 1] : (r >> 1) == 0 ? sw[0] : (r >> 1) == 1 ? sw[1] : (r >> 1) == 2 ? sw[2] : sw[3];
            d[k] = h2f((uint16_t)((r & 1) ? (word >> 16) : (word & 0xFFFFu)));
            l_dd[r * ST + jw] = HM ? half_of(m8, r) : d[k];
        }
#pragma unroll
        for (int m = 0; m < M; m++) {
            const u32x4* xs = (const u32x4*)(l_xq + (m * NB + jw) * 8);
            const u32x4 x0 = xs[0], x1 = xs[1];
            const int xq[8] = {(int)x0.x, (int)x0.y, (int)x0.z, (int)x0.w, (int)x1.x, (int)x1.y, (int)x1.z, (int)x1.w};
            const float dx = l_dx[m * NB + jw];
#pragma unroll
            for (int k = 0; k < RPT; k++) {
                const int r = sub * RPT + k;
                l_op[(m * 8 + r) * ST + jw] = (float)q4_block_dot(c[k], xq);
                l_oq[(m * 8 + r) * ST + jw] = d[k] * dx;
            }
        }
    }
    __syncthreads();
    if (t >= 64) return;
    const bool acc_lane = lane < 8 * M, cor_lane = lane >= 8 * M && lane < 16 * M;
    float chain = 0.0f;
    if (acc_lane || cor_lane) {
        const int k = acc_lane ? lane : lane - 8 * M, m = k >> 3, r = k & 7;
        const f32x4* ap = (const f32x4*)(acc_lane ? l_op + (m * 8 + r) * ST : l_dd + r * ST);
        const f32x4* bp = (const f32x4*)(acc_lane ? l_oq + (m * 8 + r) * ST : l_s + m * ST);
        const int nq = nbr / 4;
        for (int q0 = 0; q0 + 16 <= nq; q0 += 16) {   // per 64 blocks: the reads of the next 6 quads in flight
            f32x4 qa[16], qb[16];
#pragma unroll
            for (int q = 0; q < 6; q++) { qa[q] = ap[q0 + q]; qb[q] = bp[q0 + q]; }
#pragma unroll
            for (int q = 0; q < 16; q++) {
                if (q + 6 < 16) { qa[q + 6] = ap[q0 + q + 6]; qb[q + 6] = bp[q0 + q + 6]; }
                __builtin_amdgcn_sched_barrier(0);
                chain = fmaf(qa[q].x, qb[q].x, chain);
                chain = fmaf(qa[q].y, qb[q].y, chain);
                chain = fmaf(qa[q].z, qb[q].z, chain);
                chain = fmaf(qa[q].w, qb[q].w, chain);
            }
        }
        if (NR)   // the last nb % 64 blocks, in order
            for (int q = nq & ~15; q < nq; q++) {
                const f32x4 x = ap[q], y = bp[q];
                chain = fmaf(x.x, y.x, chain);
                chain = fmaf(x.y, y.y, chain);
                chain = fmaf(x.z, y.z, chain);
                chain = fmaf(x.w, y.w, chain);
            }
    }
    const float cor = __shfl(chain, (lane + 8 * M) & 63);
    if (acc_lane) {
        const int m = lane >> 3, r = lane & 7;
        a.out[(size_t)m * a.out_ld + 8 * g + r] = HALF ? chain - cor : HM ? chain + cor : fmaf(-8.0f, cor, chain);
    }
}

template <int M, bool HALF, int NB, bool HM = false, bool PRE = false, bool NR = false>
__global__ __launch_bounds__(256) void k_gemv_cut(gemv_args a) {
    gemv_cut_body<M, HALF, NB, HM, PRE, NR>(a, blockIdx.x);
}

// several tables in one launch: workgroup b computes group b - start[t] of table t (start[t] <= b < start[t + 1]),
// with the same code and operands as k_gemv_cut on that (Q4_0) table alone. NBF: the launch's one width in blocks, or 0 for
// tables of several widths (the body for the table's width chosen per workgroup, at the widest body's registers)
template <int M, bool HALF, int NBF>
__global__ __launch_bounds__(256) void k_gemv_cut_group(gemv_group_args G) {
    const int b = blockIdx.x;
    int t = 0;
#pragma unroll
    for (int i = 1; i < GEMV_GROUP_MAX; i++)
        if (i < G.n && b >= G.start[i]) t = i;
    gemv_args a{};
    a.W = G.W[t];
    a.src = G.src[t];
    a.src_ld = a.W.cols;
    a.out = G.out[t];
    a.out_ld = a.W.rows;
    const int g = b - G.start[t];
    if (NBF) gemv_cut_body<M, HALF, NBF ? NBF : 64, false>(a, g);
    else if (a.W.nb == 64) gemv_cut_body<M, HALF, 64, false>(a, g);
    else if (a.W.nb == 128) gemv_cut_body<M, HALF, 128, false>(a, g);
    else gemv_cut_body<M, HALF, 256, false>(a, g);
}

// widths the 256-block cut body takes with a runtime block count: multiples of 16 between 128 and 256
static bool nb_runtime256(int nb) { return nb > 128 && nb < 256 && nb % 16 == 0; }

static size_t gemv_cut_lds(int M, int nb) {
    const size_t st = (size_t)nb + 4;
    return sizeof(float) * ((size_t)M * nb * 8 + (size_t)M * nb + (size_t)M * st + (size_t)2 * M * 8 * st + 8 * st);
}

// ---------------------------------------------------------------- Q4_0 GEMV behind the post-norm residual
// (x += norm(y) * w_post; h = norm(x) * w_pre; imi/core/seoul.cpp:462-475, imi/core/vec.h:20-44), 512 threads per
// workgroup, a chunk of upw units (UG groups of 8 rows each) per workgroup and step of its loop:
//  - the prologue's input vectors are requested first (FFN gate|up and word scores: then half of the first chunk's
//    code rows), the rest of the chunk once y is in LDS (the whole chunk requested at kernel start, the 256
//    workgroups' weight streams held every workgroup's inputs back by about 1.5 us);
//  - prologue: the E-value vectors are read once per workgroup, one wave per conversation runs imi's AVX2-order norm
//    chains over them in LDS (held transposed, 16-byte reads: rms_scale_xt), every thread updates and normalises its
//    4 values, and the 8 threads of
//    each 32-value block cut it to int8 (imi_cut32, imi/core/vec.h:47-75: amax and code sums reduced across lanes);
//  - dots: thread (row subset, group, block) forms the exact integer dots of its rows, chain operands to LDS;
//    the next chunk's weights are requested as soon as these registers are free;
//  - chains: acc on threads 0.., cor on threads 256.. (other SIMDs), imi's per-row order
//    (imi/core/tables.cpp:127-143); epilogue: rows stored, SwiGLU of (gate, up) groups (imi/core/seoul.cpp:380-394),
//    the gated short conv of (b, c, x) groups (:407-423) or word scores with the workgroup's first maximum.
constexpr int XLD = 68;   // row stride of a transposed E <= 2048 vector: value i at (i % 32) * XLD + i / 32

// imi's norm scale of E = 256 .. 2048 values held transposed (rms_scale_xt), by one wave
__device__ __forceinline__ float rms_xt(const float* xt, int E, float eps) {
    switch (E) {
        case 256: return rms_scale_xt<2, XLD>(xt, eps);
        case 512: return rms_scale_xt<4, XLD>(xt, eps);
        case 1024: return rms_scale_xt<8, XLD>(xt, eps);
        default: return rms_scale_xt<16, XLD>(xt, eps);
    }
}

// thread t's values 4t .. 4t+3 into the transposed layout: rows 4 (t % 8) + k of column t / 8
__device__ __forceinline__ void put_xt(float* xt, int t, const f32x4& v) {
    float* p = xt + (4 * (t & 7)) * XLD + (t >> 3);
    p[0] = v.x;
    p[XLD] = v.y;
    p[2 * XLD] = v.z;
    p[3 * XLD] = v.w;
}

// values 4t .. 4t+3 of conversation m's input row: the word's dequantized row (Q4_0: (code - 8) * d; Q6_K:
// (d * scale) * (value - 32), imi/core/tables.cpp:216-233) or the given vector (imi/core/seoul.cpp:363-364)
__device__ __forceinline__ f32x4 embed_quad(const gemv_args& a, int m, int t, int E) {
    const int tok = a.P->token[m];
    if (tok < 0) return ((const f32x4*)(a.embd + (size_t)m * E))[t];
    float v[4];
    if (a.emb6.codes) {
        const int e = 4 * t, i = e >> 8, p = e & 255, h = p >> 7, k = (p >> 5) & 3, l = p & 31, sx = p >> 4;
        const size_t u = (size_t)tok * a.emb6.nbk + i;
        const unsigned* base = (const unsigned*)((const u32x4*)a.emb6.codes + (u >> 6) * 13 * 64 + (u & 63));
        const int dq = 16 * h + 8 * (k & 1) + (l >> 2), dh = 8 * h + (l >> 2);   // ql / qh dwords
        const unsigned ql = base[(dq >> 2) * 256 + (dq & 3)], qh = base[(8 + (dh >> 2)) * 256 + (dh & 3)];
        const unsigned sw = base[12 * 256 + (sx >> 2)];
        const float ds = h2f(a.emb6.d[u]) * (float)(int8_t)((sw >> (8 * (sx & 3))) & 0xFFu);
#pragma unroll
        for (int b = 0; b < 4; b++) {
            const unsigned lo = (ql >> (8 * b)) & 0xFFu, hi = (qh >> (8 * b)) & 0xFFu;
            const int q = (int)(((k < 2 ? lo : lo >> 4) & 15u) | (((hi >> (2 * k)) & 3u) << 4));
            v[b] = ds * (float)(q - 32);
        }
    } else {
        const int nb = a.emb.nb, j = t >> 3, q = t & 7;
        const u32x4 c = ((const u32x4*)a.emb.codes)[(size_t)tok * nb + j];
        const unsigned word = (q & 3) == 0 ? c.x : (q & 3) == 1 ? c.y : (q & 3) == 2 ? c.z : c.w;
        const float d = h2f(((const uint16_t*)a.emb.scales)[((size_t)(tok >> 3) * nb + j) * 8 + (tok & 7)]);
#pragma unroll
        for (int b = 0; b < 4; b++) {
            const unsigned byte = (word >> (8 * b)) & 0xFFu;
            v[b] = (float)((int)(q < 4 ? byte & 15u : byte >> 4) - 8) * d;
        }
    }
    return f32x4{v[0], v[1], v[2], v[3]};
}

// HM: Q4_1 table, as k_gemv_cut. EMB: the layer-0 form, whose input is the embedding row (no residual to add).
// RPT: rows per thread when the launch fixes it (8: a chunk of at least 5 groups of 64 blocks; the row and scale
// indices are then compile-time), 0 = from the chunk's shape
template <int M, int EPI, int UG, bool HM = false, bool EMB = false, int RPT = 0>
__global__ __launch_bounds__(512) void k_gemv_norm(gemv_args a) {
    extern __shared__ __align__(16) float lds[];
    const int E = a.E, nb = a.W.nb, st = ((nb + 3) & ~3) + 4;
    const int upw = a.upw, G = upw * UG, R = 8 * G, C = M * R;
    const int t = threadIdx.x, nq = E / 4;
    float* l_v = lds;                              // [M][32][XLD] the norm input (y, then x), transposed
    int* l_xq = (int*)(l_v + M * 32 * XLD);        // [M][nb][8] codes of the cut input
    float* l_dx = (float*)(l_xq + M * nb * 8);     // [M][nb]
    float* l_s = l_dx + M * nb;                    // [M][st]
    float* l_op = l_s + M * st;                    // [M][R][st] float(isum)
    float* l_oq = l_op + M * R * st;               // [M][R][st] d * dx
    float* l_dd = l_oq + M * R * st;               // [R][st] d
    float* l_cor = l_dd + R * st;                  // [C]
    float* l_out = l_cor + C;                      // [C]
    float* l_sc = l_out + C;                       // [16] norm scales, reduction scratch
    int* l_si = (int*)(l_sc + 16);                 // [16]
    uint64_t* l_exp = (uint64_t*)(l_si + 16);      // [32] the exponential's table (SwiGLU)
    float* l_lg = (float*)(l_exp + 32);            // word scores: [chunks of this workgroup][C], written after the loop

    const int gtot = a.W.rows / 8, nchunk = (a.units + upw - 1) / upw;
    // this thread's share of a chunk's weights: rows sub * rpt .. + rpt - 1 of group gi, block jw
    const int np = G * nb, rpt = RPT ? RPT : np <= 64 ? 1 : np <= 128 ? 2 : np <= 256 ? 4 : 8;
    const bool wt = t < np * (8 / rpt);
    const int sub = t / np, pr = t - sub * np, gi = pr / nb, jw = pr - gi * nb;
    u32x4 w[HM ? 10 : 9];
    // all 9 (Q4_1: 10) loads are issued on every path (the slots past this thread's share read the group's other rows,
    // never an address another slot reads: the compiler would fold two loads of one address into one load and a
    // register copy, and wait for the load at the copy), so the compiler counts them exactly and the prologue waits
    // only for its own inputs
    auto load_rows = [&](int k, int r0, int r1) {
        const int g = min(k * G + (wt ? gi : 0), gtot - 1), s0 = wt ? sub * rpt : 0;
        const u32x4* cp = (const u32x4*)a.W.codes + (size_t)(8 * g + s0) * nb + jw;
#pragma unroll
        for (int r = r0; r < r1; r++) w[r] = __builtin_nontemporal_load(cp + (ptrdiff_t)(((s0 + r) & 7) - s0) * nb);
        if (r1 == 8 && r0 < 8) {
            w[8] = __builtin_nontemporal_load((const u32x4*)a.W.scales + (size_t)g * nb + jw);
            if (HM) w[HM ? 9 : 8] = __builtin_nontemporal_load((const u32x4*)a.W.mins + (size_t)g * nb + jw);
        }
    };
    auto load_chunk = [&](int k) { load_rows(k, 0, 8); };
    // the word scores keep two chunks in flight: chunk k + grid lands in w2 while chunk k is worked; a chunk past the
    // table is a stand-in load of the table's first word by every lane (one cache line), so every path issues the
    // same loads and the compiler's wait counts stay exact
    u32x4 w2[HM ? 10 : 9];
    auto load_to = [&](u32x4 (&dst)[HM ? 10 : 9], int k) {
        // (rm = 1 for a chunk of the table, 0 past it; the stand-in reads word r of the table's first line: distinct
        // addresses, so no two loads fold into one)
        const int rm = k < nchunk ? 1 : 0;
        const int g = min(min(k, nchunk - 1) * G + (wt ? gi : 0), gtot - 1), s0 = wt ? sub * rpt : 0;
        const u32x4* cp = (const u32x4*)a.W.codes;
        const ptrdiff_t base = rm * ((ptrdiff_t)(8 * g + s0) * nb + jw);
#pragma unroll
        for (int r = 0; r < 8; r++)
            dst[r] = __builtin_nontemporal_load(cp + base + rm * ((ptrdiff_t)(((s0 + r) & 7) - s0) * nb) + (1 - rm) * r);
        const ptrdiff_t so = rm * ((ptrdiff_t)g * nb + jw);
        dst[8] = __builtin_nontemporal_load((const u32x4*)a.W.scales + so);
        if (HM) dst[HM ? 9 : 8] = __builtin_nontemporal_load((const u32x4*)a.W.mins + so);
    };
    // the rest of the first chunk: only this thread's own rows (rpt of them), then the scales. Loads past rpt would be
    // duplicates that each cost the address unit as much as a real 1 KB wave load (a 2-row share issued 9 loads)
    auto load_own_rows = [&](int k, int r0) {
        const int g = min(k * G + (wt ? gi : 0), gtot - 1), s0 = wt ? sub * rpt : 0;
        const u32x4* cp = (const u32x4*)a.W.codes + (size_t)(8 * g + s0) * nb + jw;
#pragma unroll
        for (int r = r0; r < 8; r++)
            if (r < rpt) w[r] = __builtin_nontemporal_load(cp + (size_t)r * nb);
        w[8] = __builtin_nontemporal_load((const u32x4*)a.W.scales + (size_t)g * nb + jw);
        if (HM) w[HM ? 9 : 8] = __builtin_nontemporal_load((const u32x4*)a.W.mins + (size_t)g * nb + jw);
    };
    // ---- prologue: its inputs are requested first, most of the weights once the inputs have arrived ----
    // (every load on every path: threads past the E / 4 quads re-read the last one, and a workgroup past the last
    // chunk loads that chunk, so the compiler's wait counts stay exact)
    f32x4 xv[M], yv[M];
    const int tq = t < nq ? t : nq - 1;
#pragma unroll
    for (int m = 0; m < M; m++) {
        if (EMB) {
            xv[m] = embed_quad(a, m, tq, E);
            yv[m] = xv[m];
        } else {
            xv[m] = ((const f32x4*)(a.x_in + (size_t)m * E))[tq];
            yv[m] = ((const f32x4*)(a.y_in + (size_t)m * E))[tq];
        }
    }
    const f32x4 wp = EMB ? f32x4{0, 0, 0, 0} : ((const f32x4*)a.w_post)[tq], wq = ((const f32x4*)a.w_pre)[tq];
    // (SwiGLU only: copied to LDS once the dots have waited for the weights. Elsewhere an unused half of the loaded
    // pair was a register the compiler reused at once, which made it wait for the inputs before the first weight
    // rows were requested)
    const uint64_t etab = EPI == EPI_SWIGLU ? kExp2Tab[t & 31] : 0;
    int k = blockIdx.x;
    if (EMB) load_chunk(k < nchunk ? k : nchunk - 1);
    // the conv epilogue's taps and memory of this thread's channel (one chunk per workgroup), right behind the inputs,
    // by the waves that hold conv channels only (the others would issue 17 clamped loads each for nothing)
    constexpr int CMAX = 8;
    float cw[CMAX + 1], cst[CMAX];
    if (EPI == EPI_CONV && __builtin_amdgcn_readfirstlane(t >> 6) < (C + 63) / 64) {
        const int m = t / R, r = t - m * R, ui = r / 24, i = r - 24 * ui, dc = a.d_conv;
        const bool mine = t < C && i < 8 && k < nchunk;
        const int e = mine ? 8 * (k * upw + ui) + i : 0;
        // both conversations' memory pointers read as uniform values, every tap and memory load issued (indices
        // clamped to the kernel's taps, unused values dropped afterwards), so the loads need no branch and the
        // compiler's wait counts stay exact
        SH_GLOBAL float* const c0 = global_ptr(a.P->conv[0]);
        SH_GLOBAL float* const c1 = M > 1 ? global_ptr(a.P->conv[M - 1]) : c0;
        const SH_GLOBAL float* stt = (mine && m ? c1 : c0) + (size_t)a.conv_layer * dc * E;
        // (taps past d_conv hold a clamped duplicate the epilogue never reads: no select here, which would wait for
        // every load right away)
#pragma unroll
        for (int q = 0; q <= CMAX; q++) cw[q] = a.conv_w[(size_t)min(q, dc) * E + e];
#pragma unroll
        for (int q = 0; q < CMAX; q++) cst[q] = stt[(size_t)min(q, dc - 1) * E + e];
    }
    // then the first kEarlyRows code rows of the first chunk, the rest (and the scales) once y is in LDS: the memory
    // system streams weights while the inputs arrive without the whole chunk queued ahead of them. Half of a thread's
    // 8 rows for the FFN gate|up and word-score tables (decode B=1 2188 -> 2211 tokens/s; 2, 3, 5, 6 or all 8 rows with
    // the scales measured no better or slower); all of a thread's rows for the q|k|v|gate table (2 at 2048 columns);
    // one of the 4 for conv in_proj, whose conv taps and memory are requested ahead of its rows (B=2 +0.2 % against
    // all 4; 2 no better)
    constexpr int kEarlyRows = (EPI == EPI_SWIGLU || EPI == EPI_LOGITS) ? 4 : EPI == EPI_CONV ? 1 : 2;
    if (!EMB) load_rows(k < nchunk ? k : nchunk - 1, 0, kEarlyRows);

    if (!EMB) {   // x += norm(y) * w_post (imi_norm_mul_add)
        if (t < nq)
#pragma unroll
            for (int m = 0; m < M; m++) put_xt(l_v + m * 32 * XLD, t, yv[m]);
        __syncthreads();
        // x, the norm weights (and the exponential's table entry) were requested with y, before any weight row:
        // taken here, so the waits for them below do not count the weight loads, whose number is this thread's row
        // count (the dots then wait for every load, as they need all of them)
#pragma unroll
        for (int m = 0; m < M; m++) asm volatile("" ::"v"(xv[m].x));
        asm volatile("" ::"v"(wp.x), "v"(wq.x), "v"((unsigned)etab));
        // (the word scores request the rest of their first chunk two rows at a time between the prologue's barriers
        // and their second chunk after the prologue: a wave cannot issue loads faster than the compute unit's earlier
        // requests drain, so 14 loads per thread ahead of the prologue's barriers held every barrier until about
        // 100 KB had arrived, 2.7 us, while two rows per phase drain within it)
        if (EPI != EPI_LOGITS) load_own_rows(k < nchunk ? k : nchunk - 1, kEarlyRows);
        else load_rows(k < nchunk ? k : nchunk - 1, kEarlyRows, 6);
        if ((t >> 6) < M) {
            const float sc = rms_xt(l_v + (t >> 6) * 32 * XLD, E, a.eps);
            if ((t & 63) == 0) l_sc[t >> 6] = sc;
        }
        __syncthreads();
#pragma unroll
        for (int m = 0; m < M; m++) {
            const float sc = l_sc[m];
            xv[m].x = fmaf(yv[m].x * sc, wp.x, xv[m].x);
            xv[m].y = fmaf(yv[m].y * sc, wp.y, xv[m].y);
            xv[m].z = fmaf(yv[m].z * sc, wp.z, xv[m].z);
            xv[m].w = fmaf(yv[m].w * sc, wp.w, xv[m].w);
        }
        // (no barrier before x overwrites y in LDS: y's only reader, the first norm, finished before the barrier above)
    }
    // (the word scores store x and the hidden state after their chunk loop: a store pending between the weight loads
    // and the dots would make the compiler wait for every load there, the next chunk's included)
    constexpr bool late_stores = EPI == EPI_LOGITS;
    f32x4 hsave[late_stores ? M : 1];
    if (EPI == EPI_LOGITS) load_rows(k < nchunk ? k : nchunk - 1, 6, 8);
    if (t < nq)
#pragma unroll
        for (int m = 0; m < M; m++) {
            put_xt(l_v + m * 32 * XLD, t, xv[m]);
            if (!late_stores && blockIdx.x == 0 && a.x_out) ((f32x4*)(a.x_out + (size_t)m * E))[t] = xv[m];
        }
    __syncthreads();
    if ((t >> 6) < M) {   // h = norm(x) * w_pre (imi_norm_mul)
        const float sc = rms_xt(l_v + (t >> 6) * 32 * XLD, E, a.eps);
        if ((t & 63) == 0) l_sc[4 + (t >> 6)] = sc;
    }
    __syncthreads();
    if (t < nq) {
        const int j = t >> 3, q = t & 7;   // block j, values 4q .. 4q+3 (8 consecutive lanes per block)
#pragma unroll
        for (int m = 0; m < M; m++) {
            const float sc = l_sc[4 + m];
            float h[4] = {xv[m].x * sc * wq.x, xv[m].y * sc * wq.y, xv[m].z * sc * wq.z, xv[m].w * sc * wq.w};
            if (late_stores) hsave[late_stores ? m : 0] = f32x4{h[0], h[1], h[2], h[3]};
            else if (a.hidden_out && blockIdx.x == 0) ((f32x4*)(a.hidden_out + (size_t)m * E))[t] = f32x4{h[0], h[1], h[2], h[3]};
            float amax = fmaxf(fmaxf(fabsf(h[0]), fabsf(h[1])), fmaxf(fabsf(h[2]), fabsf(h[3])));
            amax = fmaxf(amax, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(amax), 0xB1, 0xF, 0xF, true)));
            amax = fmaxf(amax, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(amax), 0x4E, 0xF, 0xF, true)));
            amax = fmaxf(amax, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(amax), 0x141, 0xF, 0xF, true)));
            const float d = amax / 127.0f;
            const float id = d != 0.0f ? 1.0f / d : 0.0f;
            int sum = 0;
            unsigned packed = 0;
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const int cq = (int)rintf(h[i] * id);
                sum += cq;
                packed |= ((unsigned)cq & 0xFFu) << (8 * i);
            }
            sum += __builtin_amdgcn_update_dpp(0, sum, 0xB1, 0xF, 0xF, true);
            sum += __builtin_amdgcn_update_dpp(0, sum, 0x4E, 0xF, 0xF, true);
            sum += __builtin_amdgcn_update_dpp(0, sum, 0x141, 0xF, 0xF, true);
            l_xq[(m * nb + j) * 8 + q] = (int)packed;
            if (q == 0) {
                l_dx[m * nb + j] = d;
                l_s[m * st + j] = d * (float)sum;
            }
        }
    }
    __syncthreads();
    if (EPI == EPI_LOGITS) load_to(w2, k + (int)gridDim.x);

    float best_v[M];
    int best_i[M];
#pragma unroll
    for (int m = 0; m < M; m++) { best_v[m] = -INFINITY; best_i[m] = 0x7fffffff; }
    // pf: the word scores request chunk k + 2 grid into this chunk's registers once its dots are done
    auto chunk = [&](u32x4 (&w)[HM ? 10 : 9], const int k, const int ci, const bool pf) {
        const int u0 = k * upw, g0 = k * G, gv = min(G, gtot - g0);   // groups of this chunk that exist
        // ---- dots: exact integer sums of this thread's rows, chain operands to LDS ----
        if (wt && gi < gv) {
            const unsigned sw[4] = {w[8].x, w[8].y, w[8].z, w[8].w};
            float d[8];
#pragma unroll
            for (int r = 0; r < 8; r++) {
                const int rr = (sub * rpt + r) & 7;
                const unsigned word = (rr >> 1) == 0 ? sw[0] : (rr >> 1) == 1 ? sw[1] : (rr >> 1) == 2 ? sw[2] : sw[3];
                d[r] = h2f((uint16_t)((rr & 1) ? (word >> 16) : (word & 0xFFFFu)));
            }
            const int r0 = 8 * gi + sub * rpt;
#pragma unroll
            for (int r = 0; r < 8; r++)
                if (r < rpt) l_dd[(r0 + r) * st + jw] = HM ? half_of(w[HM ? 9 : 8], (sub * rpt + r) & 7) : d[r];
#pragma unroll
            for (int m = 0; m < M; m++) {
                const u32x4* xs = (const u32x4*)(l_xq + (m * nb + jw) * 8);
                const u32x4 x0 = xs[0], x1 = xs[1];
                const int xq[8] = {(int)x0.x, (int)x0.y, (int)x0.z, (int)x0.w, (int)x1.x, (int)x1.y, (int)x1.z, (int)x1.w};
                const float dx = l_dx[m * nb + jw];
#pragma unroll
                for (int r = 0; r < 8; r++)
                    if (r < rpt) {
                        l_op[(m * R + r0 + r) * st + jw] = (float)q4_block_dot(w[r], xq);
                        l_oq[(m * R + r0 + r) * st + jw] = d[r] * dx;
                    }
            }
        }
        if (EPI == EPI_SWIGLU && t < 32) l_exp[t] = etab;
        __syncthreads();
        if (EPI == EPI_LOGITS && pf) load_to(w, k + 2 * (int)gridDim.x);   // in flight during this and the next chunk
        // ---- chains ----
        const bool acc_lane = t < C, cor_lane = t >= 256 && t - 256 < C;
        float chain = 0.0f;
        const int c = acc_lane ? t : t - 256;
        if ((acc_lane || cor_lane) && (c % R) < 8 * gv) {
            const int m = c / R, r = c - m * R;
            const f32x4* ap = (const f32x4*)(acc_lane ? l_op + (m * R + r) * st : l_dd + r * st);
            const f32x4* bp = (const f32x4*)(acc_lane ? l_oq + (m * R + r) * st : l_s + m * st);
            if ((nb & 63) == 0) {
                for (int q0 = 0; q0 < nb / 4; q0 += 16) {
                    f32x4 qa[16], qb[16];
#pragma unroll
                    for (int q = 0; q < 6; q++) { qa[q] = ap[q0 + q]; qb[q] = bp[q0 + q]; }
#pragma unroll
                    for (int q = 0; q < 16; q++) {
                        if (q + 6 < 16) { qa[q + 6] = ap[q0 + q + 6]; qb[q + 6] = bp[q0 + q + 6]; }
                        __builtin_amdgcn_sched_barrier(0);
                        chain = fmaf(qa[q].x, qb[q].x, chain);
                        chain = fmaf(qa[q].y, qb[q].y, chain);
                        chain = fmaf(qa[q].z, qb[q].z, chain);
                        chain = fmaf(qa[q].w, qb[q].w, chain);
                    }
                }
            } else {
                const float* as = (const float*)ap;
                const float* bs = (const float*)bp;
                for (int q = 0; q < nb; q++) chain = fmaf(as[q], bs[q], chain);
            }
            if (cor_lane) l_cor[c] = chain;
        }
        __syncthreads();
        // the row's value stays in the acc lane's register. The conv epilogue reads rows 8 and 16 lanes on, across a
        // wave's end, through LDS and a barrier; a SwiGLU gate row (lane i < 8 of a 16-lane unit, units aligned to 16
        // lanes) takes its up row from lane i + 8 of the same DPP row, a shift computed by every lane outside the
        // branches (the register pin keeps the compiler from folding the shift into a user under a narrower mask)
        const float outv = acc_lane ? (HM ? chain + l_cor[c] : fmaf(-8.0f, l_cor[c], chain)) : 0.0f;
        float upv = 0.0f;
        if (EPI == EPI_SWIGLU) {
            upv = __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(outv), 0x108, 0xF, 0xF, true));
            asm volatile("" : "+v"(upv));
        }
        if (EPI == EPI_CONV) {
            if (acc_lane) l_out[c] = outv;
            __syncthreads();
        }
        // ---- epilogue: thread c < C holds row r of the chunk for input m ----
        float act = 0.0f;   // EPI_SWIGLU: this thread's channel output (threads on up rows: 0)
        if (t < C) {
            const int m = t / R, r = t - m * R;
            const float v = outv;
            if (r < 8 * gv) {
                if (EPI == EPI_STORE) {
                    a.out[(size_t)m * a.out_ld + 8 * g0 + r] = v;
                } else if (EPI == EPI_SWIGLU) {   // unit = (gate group, up group) of 8 channels
                    const int ui = r >> 4, i = r & 15;
                    if (i < 8) {
                        act = silu_t(v, (const uint64_t*)l_exp) * upv;
                        a.out[(size_t)m * a.out_ld + 8 * (u0 + ui) + i] = act;
                    }
                } else if (EPI == EPI_CONV) {     // unit = (b, c, x) groups of 8 channels
                    const int ui = r / 24, i = r - 24 * ui;
                    if (i < 8) {
                        const int e = 8 * (u0 + ui) + i, dc = a.d_conv;
                        const float cc = l_out[t + 8], xx = l_out[t + 16];
                        SH_GLOBAL float* stt = global_ptr(a.P->conv[m]) + (size_t)a.conv_layer * dc * E;
                        const float bx = v * xx;
                        float wdc = cw[0];
#pragma unroll
                        for (int q = 1; q <= CMAX; q++)
                            if (q == dc) wdc = cw[q];
                        float uu = v * xx * wdc;
#pragma unroll
                        for (int q = 0; q < CMAX; q++)
                            if (q < dc) uu = fmaf(cst[q], cw[q], uu);
                        uu *= cc;
#pragma unroll
                        for (int q = 0; q + 1 < CMAX; q++)
                            if (q + 1 < dc) stt[(size_t)q * E + e] = cst[q + 1];
                        stt[(size_t)(dc - 1) * E + e] = bx;
                        a.out[(size_t)m * a.out_ld + e] = uu;
                    }
                } else {   // EPI_LOGITS
                    const int row = 8 * g0 + r;
                    if (a.out) l_lg[ci * C + t] = v;   // (to the output after the chunk loop)
#pragma unroll
                    for (int mm = 0; mm < M; mm++)
                        if (mm == m && (v > best_v[mm] || (v == best_v[mm] && row < best_i[mm]))) { best_v[mm] = v; best_i[mm] = row; }
                }
            }
        }
        // the next table's input cut here (imi_cut32, imi/core/vec.h:47-75): with 4 units per chunk, wave m holds
        // conversation m's 32 channels of this chunk (one cut block); amax and the code sum are order-free reductions,
        // d = amax / 127, id = d ? 1 / d : 0, q = rint(x * id), s = d * sum, as the cut in the next kernel's prologue
        if (EPI == EPI_SWIGLU && a.outq && t < C) {
            // the block's channels sit in lanes 16 j + i (i < 8) of the wave: 8-lane reductions by DPP, then the four
            // groups' lanes 0, 16, 32, 48 read as scalars
            float am = fabsf(act);
            am = fmaxf(am, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(am), 0xB1, 0xF, 0xF, true)));
            am = fmaxf(am, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(am), 0x4E, 0xF, 0xF, true)));
            am = fmaxf(am, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(am), 0x141, 0xF, 0xF, true)));
            const int ai = __float_as_int(am);
            const float amax = fmaxf(fmaxf(__int_as_float(__builtin_amdgcn_readlane(ai, 0)), __int_as_float(__builtin_amdgcn_readlane(ai, 16))),
                                     fmaxf(__int_as_float(__builtin_amdgcn_readlane(ai, 32)), __int_as_float(__builtin_amdgcn_readlane(ai, 48))));
            const float d = amax / 127.0f;
            const float id = d != 0.0f ? 1.0f / d : 0.0f;
            const int q = (int)rintf(act * id);
            int sq = q;
            sq += __builtin_amdgcn_update_dpp(0, sq, 0xB1, 0xF, 0xF, true);
            sq += __builtin_amdgcn_update_dpp(0, sq, 0x4E, 0xF, 0xF, true);
            sq += __builtin_amdgcn_update_dpp(0, sq, 0x141, 0xF, 0xF, true);
            const int sum = (__builtin_amdgcn_readlane(sq, 0) + __builtin_amdgcn_readlane(sq, 16)) +
                            (__builtin_amdgcn_readlane(sq, 32) + __builtin_amdgcn_readlane(sq, 48));
            const int m = t / R, r = t - m * R, ui = r >> 4, i = r & 15;
            const int nblk = a.out_ld / 32;
            if (i < 8) a.outq[(size_t)m * a.out_ld + 8 * (u0 + ui) + i] = (int8_t)q;
            if ((t & 63) == 0) {
                a.outd[(size_t)m * nblk + u0 / 4] = d;
                a.outs[(size_t)m * nblk + u0 / 4] = d * (float)sum;
            }
        }
        __syncthreads();
    };
    if (EPI == EPI_LOGITS) {   // chunks k, k + grid, ... alternating between the two register sets
        int ci = 0;
        // the first six chunks straight-line (a word table of 97,496 rows gives a workgroup at most six): inside a
        // loop the compiler waits for every load at the first use of a chunk's registers, the next chunk's included.
        // The last two request nothing (a request past the table would be a stand-in load that the kernel's end
        // waits for)
#pragma unroll
        for (int it = 0; it < 6; it++) {
            if (k >= nchunk) break;
            if (it & 1) chunk(w2, k, ci++, it < 4);
            else chunk(w, k, ci++, it < 4);
            k += gridDim.x;
        }
        if (k < nchunk) {   // (larger tables: the rest in a loop, two chunks in flight again)
            load_to(w, k);
            load_to(w2, k + (int)gridDim.x);
            for (;;) {
                if (k >= nchunk) break;
                chunk(w, k, ci++, true);
                k += gridDim.x;
                if (k >= nchunk) break;
                chunk(w2, k, ci++, true);
                k += gridDim.x;
            }
        }
        // the scores kept in LDS (stores in the loop would leave the compiler unable to wait for just the older chunk)
        if (a.out && t < C) {
            const int m = t / R, r = t - m * R;
            for (int c2 = 0; c2 < ci; c2++) {
                const int g0 = ((int)blockIdx.x + c2 * (int)gridDim.x) * G;
                if (r < 8 * min(G, gtot - g0)) a.out[(size_t)m * a.out_ld + 8 * g0 + r] = l_lg[c2 * C + t];
            }
        }
    } else if (k < nchunk) {   // (every other table: one chunk per workgroup)
        chunk(w, k, 0, false);
    }
    if (late_stores && blockIdx.x == 0 && t < nq)
#pragma unroll
        for (int m = 0; m < M; m++) {
            if (a.x_out) ((f32x4*)(a.x_out + (size_t)m * E))[t] = xv[m];
            if (a.hidden_out) ((f32x4*)(a.hidden_out + (size_t)m * E))[t] = hsave[late_stores ? m : 0];
        }
    if (EPI == EPI_LOGITS) {   // the workgroup's first maximum per input
#pragma unroll
        for (int m = 0; m < M; m++) {
            float v = best_v[m];
            int i = best_i[m];
#pragma unroll
            for (int o = 32; o > 0; o >>= 1) {
                const float ov = __shfl_xor(v, o);
                const int oi = __shfl_xor(i, o);
                if (ov > v || (ov == v && oi < i)) { v = ov; i = oi; }
            }
            if ((t & 63) == 0) { l_sc[8 + (t >> 6)] = v; l_si[8 + (t >> 6)] = i; }
            __syncthreads();
            if (t == 0) {
                float bv = l_sc[8];
                int bi = l_si[8];
                for (int q = 1; q < 8; q++)
                    if (l_sc[8 + q] > bv || (l_sc[8 + q] == bv && l_si[8 + q] < bi)) { bv = l_sc[8 + q]; bi = l_si[8 + q]; }
                a.part_v[m * gridDim.x + blockIdx.x] = bv;
                a.part_i[m * gridDim.x + blockIdx.x] = bi;
            }
            __syncthreads();
        }
    }
}

// chunks_per_wg: the word scores' chunks per workgroup (their scores wait in LDS until the chunk loop ends), else 0
static size_t gemv_norm_lds(int M, int E, int nb, int G, int chunks_per_wg = 0) {
    const size_t st = (size_t)(((nb + 3) & ~3) + 4), R = 8 * (size_t)G, C = M * R;
    (void)E;
    return sizeof(float) * ((size_t)M * 32 * XLD + (size_t)M * nb * 8 + (size_t)M * nb + M * st + 2 * M * R * st + R * st + 2 * C + 32 + 64 +
                            (size_t)chunks_per_wg * C);
}

// ---------------------------------------------------------------- word scores over a Q6_K table
// imi/core/seoul.cpp:479-487: the hidden state cut per 256 values (imi_q8k::from, imi/core/tables.cpp:200-213) and
// each row scored by imi_q6k_row (tables.cpp:235-277) in its AVX2 op order. 512 threads.
//  - prologue (workgroup): h = norm(x + norm(y) * w_post) * w_pre with k_gemv_norm's norm order (block 0 writes x and
//    h), or h = src when a.src is set; thread t holds values 4t .. 4t+3, so wave b holds 256-value block b: amax by
//    wave reduction, codes rint(h / d) (half-even, as lrintf), code sums per 16 values over 4 lanes; codes, d and the
//    sums go to LDS;
//  - main loop (wave-local): a wave takes tiles of 64 units (64 / nbk rows x nbk blocks), lane = unit, and requests
//    the next tile's 13 words before the current tile's math. A lane forms its block's eight int32 AVX2 lanes: lane L
//    takes values 4L .. 4L+3 of each 32-value chunk (h, k) as one sdot4 of 6-bit values (nibble | 2 high bits) and
//    codes, times the chunk's scale for its register half (8h + 2k + L / 4), minus 32 (sc[2L] bsum[2L] +
//    sc[2L+1] bsum[2L+1]); exact. Their floats and dd = d * X.d go to LDS; 8 lanes per row then run the chains
//    acc_L = fma(dd_i, lane_iL, acc_L) over the row's blocks in order and the 256-bit horizontal sum
//    ((a0 + a4) + (a2 + a6)) + ((a1 + a5) + (a3 + a7)) by xor-shuffles 4, 2, 1 (each add commutes);
//  - the first maximum per input over the workgroup's rows goes to part_v / part_i for k_final.
namespace q6k_detail {
constexpr int XS = 68;   // LDS dwords per 256-code block (64 + 4, so the 8 blocks a wave reads sit in distinct banks)
constexpr int NW = 13;   // 16-byte words per unit
}  // namespace q6k_detail

template <int M>
__global__ __launch_bounds__(512) void k_scores_q6k(gemv_args a) {
    using namespace q6k_detail;
    extern __shared__ __align__(16) float lds[];
    constexpr int LNS = 9 * M + 1;                         // floats per unit in the lane buffer (odd stride)
    const int E = a.E, nbk = E / 256, t = threadIdx.x, lane = t & 63, wv = t >> 6, nq = E / 4;
    float* l_v = lds;                                      // [M][32][XLD] transposed norm input
    int* l_xq = (int*)(l_v + M * 32 * XLD);                // [M][nbk][XS] codes, 4 per dword
    float* l_xd = (float*)(l_xq + M * nbk * XS);           // [M][nbk]
    int* l_bs = (int*)(l_xd + M * nbk);                    // [M][nbk][16]
    float* l_sc = (float*)(l_bs + M * nbk * 16);           // [16] norm scales, reduction scratch
    int* l_si = (int*)(l_sc + 16);                         // [16]
    float* l_ln = (float*)(l_si + 16) + wv * 64 * LNS;     // this wave's [64][LNS]: lanes of m, then dd of m

    const int rows = a.W6.rows, nunit = rows * nbk, ntile = (nunit + 63) / 64;
    const u32x4* codes = (const u32x4*)a.W6.codes;
    int tile = blockIdx.x * 8 + wv;
    const int tstep = gridDim.x * 8;
    // ---- prologue: its inputs requested first, by loads on every path (operands a call does not give re-read the
    // first input, unused): a conditional load left the compiler waiting for every earlier load, and the first
    // tile's weights (about 100 KB per workgroup) requested ahead of the inputs held them back ----
    const int tq = t < nq ? t : nq - 1;
    const float* const xb = a.src ? a.src : a.x_in;
    const size_t xld = a.src ? (size_t)a.src_ld : (size_t)E;
    const float* const yb = a.y_in ? a.y_in : xb;
    const size_t yld = a.y_in ? (size_t)E : xld;
    f32x4 xv[M], yv[M];
#pragma unroll
    for (int m = 0; m < M; m++) {
        xv[m] = ((const f32x4*)(xb + (size_t)m * xld))[tq];
        yv[m] = ((const f32x4*)(yb + (size_t)m * yld))[tq];
    }
    const f32x4 wq = ((const f32x4*)(a.w_pre ? a.w_pre : xb))[tq];
    const f32x4 wp = ((const f32x4*)(a.w_post ? a.w_post : xb))[tq];
    __builtin_amdgcn_sched_barrier(0);   // (the tile's loads stay behind the inputs')
    u32x4 w[NW];
    auto load_tile = [&](int tl) {   // (a wave past the last tile re-reads the last one)
        const u32x4* b = codes + (size_t)min(tl, ntile - 1) * NW * 64 + lane;
#pragma unroll
        for (int q = 0; q < NW; q++) w[q] = __builtin_nontemporal_load(b + q * 64);
    };
    load_tile(tile);
    float dw = h2f(a.W6.d[(size_t)min(tile, ntile - 1) * 64 + lane]);

    f32x4 hv[M];
    if (a.src) {
#pragma unroll
        for (int m = 0; m < M; m++) hv[m] = xv[m];
    } else {
        if (a.y_in) {   // x += norm(y) * w_post (imi_norm_mul_add)
            if (t < nq)
#pragma unroll
                for (int m = 0; m < M; m++) put_xt(l_v + m * 32 * XLD, t, yv[m]);
            __syncthreads();
            if ((t >> 6) < M) {
                const float sc = rms_xt(l_v + (t >> 6) * 32 * XLD, E, a.eps);
                if ((t & 63) == 0) l_sc[t >> 6] = sc;
            }
            __syncthreads();
#pragma unroll
            for (int m = 0; m < M; m++) {
                const float sc = l_sc[m];
                xv[m].x = fmaf(yv[m].x * sc, wp.x, xv[m].x);
                xv[m].y = fmaf(yv[m].y * sc, wp.y, xv[m].y);
                xv[m].z = fmaf(yv[m].z * sc, wp.z, xv[m].z);
                xv[m].w = fmaf(yv[m].w * sc, wp.w, xv[m].w);
            }
            __syncthreads();
        }
        if (t < nq)
#pragma unroll
            for (int m = 0; m < M; m++) {
                put_xt(l_v + m * 32 * XLD, t, xv[m]);
                if (blockIdx.x == 0 && a.x_out) ((f32x4*)(a.x_out + (size_t)m * E))[t] = xv[m];
            }
        __syncthreads();
        if ((t >> 6) < M) {   // h = norm(x) * w_pre (imi_norm_mul)
            const float sc = rms_xt(l_v + (t >> 6) * 32 * XLD, E, a.eps);
            if ((t & 63) == 0) l_sc[4 + (t >> 6)] = sc;
        }
        __syncthreads();
#pragma unroll
        for (int m = 0; m < M; m++) {
            const float sc = l_sc[4 + m];
            hv[m] = f32x4{xv[m].x * sc * wq.x, xv[m].y * sc * wq.y, xv[m].z * sc * wq.z, xv[m].w * sc * wq.w};
            if (a.hidden_out && blockIdx.x == 0 && t < nq) ((f32x4*)(a.hidden_out + (size_t)m * E))[t] = hv[m];
        }
    }
    if (t < nq) {   // cut per 256 values: block wv, values 4 lane .. 4 lane + 3
#pragma unroll
        for (int m = 0; m < M; m++) {
            const float h[4] = {hv[m].x, hv[m].y, hv[m].z, hv[m].w};
            const float amax = wave_max(fmaxf(fmaxf(fabsf(h[0]), fabsf(h[1])), fmaxf(fabsf(h[2]), fabsf(h[3]))));
            const float d = amax / 127.0f, id = d != 0.0f ? 1.0f / d : 0.0f;
            int sum = 0;
            unsigned packed = 0;
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const int c = (int)rintf(h[i] * id);
                sum += c;
                packed |= ((unsigned)c & 0xFFu) << (8 * i);
            }
            sum += __builtin_amdgcn_update_dpp(0, sum, 0xB1, 0xF, 0xF, true);   // lanes xor 1
            sum += __builtin_amdgcn_update_dpp(0, sum, 0x4E, 0xF, 0xF, true);   // lanes xor 2
            l_xq[(m * nbk + wv) * XS + lane] = (int)packed;
            if ((lane & 3) == 0) l_bs[(m * nbk + wv) * 16 + (lane >> 2)] = sum;
            if (lane == 0) l_xd[m * nbk + wv] = d;
        }
    }
    __syncthreads();

    // ---- main loop ----
    const int bi = lane % nbk, rpt = 64 / nbk;              // this lane's block within its row; rows per tile
    float best_v[M];
    int best_i[M];
#pragma unroll
    for (int m = 0; m < M; m++) { best_v[m] = -INFINITY; best_i[m] = 0x7fffffff; }
    for (; tile < ntile; tile += tstep) {
        u32x4 c[NW];
#pragma unroll
        for (int q = 0; q < NW; q++) c[q] = w[q];
        const float d = dw;
        load_tile(tile + tstep);
        dw = h2f(a.W6.d[(size_t)min(tile + tstep, ntile - 1) * 64 + lane]);
        unsigned ql[32], qh[16];
#pragma unroll
        for (int q = 0; q < 8; q++) { ql[4 * q] = c[q].x; ql[4 * q + 1] = c[q].y; ql[4 * q + 2] = c[q].z; ql[4 * q + 3] = c[q].w; }
#pragma unroll
        for (int q = 0; q < 4; q++) { qh[4 * q] = c[8 + q].x; qh[4 * q + 1] = c[8 + q].y; qh[4 * q + 2] = c[8 + q].z; qh[4 * q + 3] = c[8 + q].w; }
        const unsigned scw[4] = {c[12].x, c[12].y, c[12].z, c[12].w};
        int sc[16];
#pragma unroll
        for (int s = 0; s < 16; s++) sc[s] = (int)(int8_t)((scw[s >> 2] >> (8 * (s & 3))) & 0xFFu);
#pragma unroll
        for (int m = 0; m < M; m++) {
            const int* xb = l_xq + (m * nbk + bi) * XS;
            const int* bs = l_bs + (m * nbk + bi) * 16;
            int isum[8];
#pragma unroll
            for (int L = 0; L < 8; L++) isum[L] = -32 * (sc[2 * L] * bs[2 * L] + sc[2 * L + 1] * bs[2 * L + 1]);
#pragma unroll
            for (int hh = 0; hh < 2; hh++)
#pragma unroll
                for (int k = 0; k < 4; k++) {
                    const u32x4 x0 = *(const u32x4*)(xb + 32 * hh + 8 * k), x1 = *(const u32x4*)(xb + 32 * hh + 8 * k + 4);
                    const unsigned xw[8] = {x0.x, x0.y, x0.z, x0.w, x1.x, x1.y, x1.z, x1.w};
#pragma unroll
                    for (int L = 0; L < 8; L++) {
                        const unsigned lo = ql[16 * hh + 8 * (k & 1) + L], hi = qh[8 * hh + L];
                        const unsigned q = ((k < 2 ? lo : lo >> 4) & 0x0F0F0F0Fu) | (((hi >> (2 * k)) & 0x03030303u) << 4);
                        isum[L] += sc[8 * hh + 2 * k + (L >> 2)] * __builtin_amdgcn_sdot4((int)q, (int)xw[L], 0, false);
                    }
                }
            float* ln = l_ln + lane * LNS + 9 * m;
#pragma unroll
            for (int L = 0; L < 8; L++) ln[L] = (float)isum[L];
            ln[8] = d * l_xd[m * nbk + bi];
        }
        __builtin_amdgcn_wave_barrier();
        for (int ci = lane; ci < rpt * 8; ci += 64) {
            const int r = ci >> 3, L = ci & 7, row = tile * rpt + r;
#pragma unroll
            for (int m = 0; m < M; m++) {
                float acc = 0.0f;
                for (int i = 0; i < nbk; i++) {
                    const float* ln = l_ln + (r * nbk + i) * LNS + 9 * m;
                    acc = fmaf(ln[8], ln[L], acc);
                }
                acc += __shfl_xor(acc, 4);
                acc += __shfl_xor(acc, 2);
                acc += __shfl_xor(acc, 1);
                if (L == 0 && row < rows) {
                    if (a.out) a.out[(size_t)m * a.out_ld + row] = acc;
                    if (acc > best_v[m] || (acc == best_v[m] && row < best_i[m])) { best_v[m] = acc; best_i[m] = row; }
                }
            }
        }
        __builtin_amdgcn_wave_barrier();
    }
    // ---- the workgroup's first maximum per input ----
#pragma unroll
    for (int m = 0; m < M; m++) {
        float v = best_v[m];
        int i = best_i[m];
#pragma unroll
        for (int o = 32; o > 0; o >>= 1) {
            const float ov = __shfl_xor(v, o);
            const int oi = __shfl_xor(i, o);
            if (ov > v || (ov == v && oi < i)) { v = ov; i = oi; }
        }
        if (lane == 0) { l_sc[8 + wv] = v; l_si[8 + wv] = i; }
        __syncthreads();
        if (t == 0) {
            float bv = l_sc[8];
            int bj = l_si[8];
            for (int q = 1; q < 8; q++)
                if (l_sc[8 + q] > bv || (l_sc[8 + q] == bv && l_si[8 + q] < bj)) { bv = l_sc[8 + q]; bj = l_si[8 + q]; }
            a.part_v[m * gridDim.x + blockIdx.x] = bv;
            a.part_i[m * gridDim.x + blockIdx.x] = bj;
        }
        __syncthreads();
    }
}

static size_t scores_q6k_lds(int M, int E) {
    const size_t nbk = (size_t)E / 256;
    return sizeof(float) * ((size_t)M * 32 * XLD + (size_t)M * nbk * (q6k_detail::XS + 1 + 16) + 32 + 8 * 64 * (9 * (size_t)M + 1));
}

// dynamic LDS bytes of a k_gemv instantiation
static size_t gemv_lds(int M, int UG, int nb, int E, bool norm) {
    const int R = 8 * UG;
    return sizeof(float) * ((size_t)nb * (M * R + 1) + 2 * (size_t)nb * (R + 1) + 2 * (size_t)M * nb + (norm ? (size_t)E : 0));
}

// ---------------------------------------------------------------- GQA decode attention
// Block per (key/value head g, conversation m), 256 threads, imi/core/seoul.cpp:433-453 in the CPU's op order:
// k = rope(norm(k) * k_norm) and v go to the fp16 cache at pos; per query head: q = rope(norm(q) * q_norm);
// score_t = dot_h(q, K_t) / sqrt(D); softmax with the max subtracted, glibc's expf and a double sum in order;
// o = sum_t fma((e_t * inv), V_t, o) in order over t; times the sigmoid head gate.
template <int D>
__global__ __launch_bounds__(256) void k_attn(attn_args a) {
    extern __shared__ float lds[];
    const int g = blockIdx.x, m = blockIdx.y, tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    constexpr int half = D / 2;
    const int Hq = a.n_head * D, kvd = a.n_kv * D, grp = a.n_head / a.n_kv;
    const int pos = a.P->pos[m];
    const int s0 = a.n_swa > 0 ? max(0, pos - a.n_swa + 1) : 0, nk = pos - s0 + 1;
    SH_GLOBAL uint16_t* kc = global_ptr(a.P->kc[m]) + ((size_t)a.layer_ai * a.n_kv + g) * a.n_ctx * D;
    SH_GLOBAL uint16_t* vc = global_ptr(a.P->vc[m]) + ((size_t)a.layer_ai * a.n_kv + g) * a.n_ctx * D;
    const float* row = a.qkv + (size_t)m * a.ld_qkv;
    float* q_s = lds;                               // [grp][D]
    float* sc = q_s + grp * D;                      // [grp][n_ctx]
    float* scratch = sc + (size_t)grp * a.n_ctx;    // [5][D]: per-wave norm staging, then the new key
    float* inv_s = scratch + 5 * D;                 // [grp]
    const float2* cs = a.rope_cs + (size_t)pos * half;

    // norm + NEOX rope of one head vector (imi/core/seoul.cpp:19-28 with the host's cos/sin table), one wave
    auto norm_rope = [&](const float* src, const float* w, float* dst) {
        float* st = scratch + wv * D;
        const float x = lane < D ? src[lane] : 0.0f;
        if (lane < D) st[lane] = x;
        __builtin_amdgcn_wave_barrier();
        const float s = rms_scale_wave(st, D, a.eps);
        const float n = lane < D ? x * s * w[lane] : 0.0f;
        const float other = __shfl(n, lane < half ? lane + half : lane - half);
        if (lane < D) {
            const float2 t = cs[lane < half ? lane : lane - half];
            dst[lane] = lane < half ? fmaf(n, t.x, -(other * t.y)) : fmaf(other, t.y, n * t.x);
        }
        __builtin_amdgcn_wave_barrier();
    };
    for (int hh = wv; hh < grp; hh += 4) norm_rope(row + (g * grp + hh) * D, a.q_norm, q_s + hh * D);
    if (wv == 0) {
        float* kd = scratch + 4 * D;
        norm_rope(row + Hq + g * D, a.k_norm, kd);
        if (lane < D) {
            kc[(size_t)pos * D + lane] = f2h(kd[lane]);
            vc[(size_t)pos * D + lane] = f2h(row[Hq + kvd + g * D + lane]);
        }
    }
    __syncthreads();

    const float scale = 1.0f / sqrtf((float)D);
    for (int t = tid; t < nk; t += 256) {
        const SH_GLOBAL uint16_t* kt = kc + (size_t)(s0 + t) * D;
        float kf[D];
#pragma unroll
        for (int i0 = 0; i0 < D; i0 += 8) {
            const u32x4 kw = *(const u32x4*)(kt + i0);
            const unsigned w4[4] = {kw.x, kw.y, kw.z, kw.w};
#pragma unroll
            for (int e = 0; e < 8; e++) kf[i0 + e] = h2f((uint16_t)((w4[e >> 1] >> (16 * (e & 1))) & 0xFFFFu));
        }
        for (int hh = 0; hh < grp; hh++) sc[(size_t)hh * a.n_ctx + t] = dot_h8<D>(q_s + hh * D, kf) * scale;
    }
    __syncthreads();
    for (int hh = wv; hh < grp; hh += 4) {
        float* s = sc + (size_t)hh * a.n_ctx;
        float mx = -INFINITY;
        for (int t = lane; t < nk; t += 64) mx = fmaxf(mx, s[t]);
        mx = wave_max(mx);
        for (int t = lane; t < nk; t += 64) s[t] = expf_glibc(s[t] - mx);
        __builtin_amdgcn_wave_barrier();
        if (lane == 0) {   // double sum in position order, as imi's loop
            double sum = 0.0;
            for (int t = 0; t < nk; t++) sum += (double)s[t];
            inv_s[hh] = (float)(1.0 / sum);
        }
    }
    __syncthreads();
    for (int k = tid; k < grp * D; k += 256) {
        const int hh = k / D, i = k - hh * D;
        const float* s = sc + (size_t)hh * a.n_ctx;
        const float inv = inv_s[hh];
        float o = 0.0f;
        for (int t = 0; t < nk; t++) o = fmaf(s[t] * inv, h2f(vc[(size_t)(s0 + t) * D + i]), o);
        const int h = g * grp + hh;
        const float gate = 1.0f / (1.0f + expf_glibc(-row[Hq + 2 * kvd + h]));
        a.att[(size_t)m * Hq + h * D + i] = o * gate;
    }
}

// ---------------------------------------------------------------- GQA decode attention, one query head per block
// Block (query head h, conversation m), 512 threads, imi/core/seoul.cpp:433-453 in the CPU's op order.
//  - requests first: each thread's first two key rows (cache rows of earlier steps) and, on waves 4-7, the first
//    value tile;
//  - q = rope(norm(q) * q_norm) (wave 0); this position's k = rope(norm(k) * k_norm) and v (wave 1; the first head
//    of each kv group writes them to the fp16 cache, the group's other heads use their own copy, the same number);
//  - score_t = dot_h(q, K_t) / sqrt(D), thread per position, the next key row requested before the current dot;
//  - softmax: max, e_t = glibc expf(s_t - max), and the double sum of e_t in position order. When every e_t is a
//    multiple of 2^(B - 51), B = floor(log2(sum)), every partial sum in any order is exact (a multiple of that unit
//    below 2^(B + 2) has at most 53 significant bits), so the in-order double sum equals the block's tree sum; else
//    wave 0 adds in position order. The maximum and the sums reduce within each wave by DPP; inv = 1 / sum is
//    formed on wave 0 alone, which needs it;
//  - a_t = e_t * inv; o = fma(a_t, V_t, o) in order over t by lane i of wave 0 (one chain per dimension, a_t formed
//    as the chain reads e_t). Waves 4-7 stage value tiles of 256 positions into LDS transposed (dimension-major,
//    16-byte slots XOR-swizzled so that both the staging writes and the chain's 8-position reads are free of bank
//    conflicts), double-buffered: tile 0 is written during the scores, tile j + 1 written and tile j + 2 requested
//    while wave 0 runs tile j;
//  - times the sigmoid head gate.
namespace attn_detail {
constexpr int NT = 512;                                        // threads
template <int D> constexpr int tile_positions() { return D > 64 ? 128 : 256; }   // value tile: 32 KB of fp16 at D 64 / 128
__device__ __forceinline__ int vswz(int d) { return (2 * (d >> 3) + 4 * (d & 7) + ((d & 7) >> 2)) & 15; }
// lowest set bit exponent of a positive float (e = 0 gives a large value)
__device__ __forceinline__ int low_bit_exp(float e) {
    const unsigned b = __float_as_uint(e), ex = b >> 23, mt = b & 0x7FFFFFu;
    if (b == 0) return 1 << 20;
    return ex == 0 ? -149 + __builtin_ctz(mt) : (int)ex - 150 + __builtin_ctz(mt | 0x800000u);
}
}  // namespace attn_detail

template <int D>
__global__ __launch_bounds__(512) void k_attn_head(attn_args a) {
    using namespace attn_detail;
    constexpr int TV = tile_positions<D>();
    constexpr int half = D / 2, KW = D / 8;        // 16-byte words per cache row
    constexpr int DPL = (D + 63) / 64;             // dimensions per lane in the per-head wave work (lane + 64 c)
    constexpr bool AHEAD2 = false;                 // key rows two passes ahead (registers: the value tile comes first)
    constexpr int NL = (TV / 8) * KW;              // loader threads: one 8-position x 8-dimension block each
    static_assert(NL <= 256 && TV / 8 <= 32, "value staging layout");
    extern __shared__ __align__(16) float lds[];
    const int h = blockIdx.x, m = blockIdx.y, t = threadIdx.x, lane = t & 63, wv = t >> 6;
    const int grp = a.n_head / a.n_kv, g = h / grp, hh = h - g * grp;
    const int Hq = a.n_head * D, kvd = a.n_kv * D;
    const int pos = a.P->pos[m];
    const int s0 = a.n_swa > 0 ? max(0, pos - a.n_swa + 1) : 0, nk = pos - s0 + 1;
    const int ntile = (nk + TV - 1) / TV;
    SH_GLOBAL uint16_t* kc = global_ptr(a.P->kc[m]) + ((size_t)a.layer_ai * a.n_kv + g) * a.n_ctx * D;
    SH_GLOBAL uint16_t* vc = global_ptr(a.P->vc[m]) + ((size_t)a.layer_ai * a.n_kv + g) * a.n_ctx * D;
    const float* row = a.qkv + (size_t)m * a.ld_qkv;
    float* q_s = lds;                              // [D]
    float* k_s = q_s + D;                          // [D] this position's key as the cache holds it
    float* red = k_s + D;                          // [32]
    double* red_d = (double*)(red + 32);           // [8]
    int* red_i = (int*)(red_d + 8);                // [8]
    uint64_t* etab = (uint64_t*)(red_i + 8);       // [32] expf's table (an LDS copy: no memory round trip in the softmax)
    float* stg = (float*)(etab + 32);              // [2][D] norm staging of waves 0 and 1
    float* sc = stg + 2 * D;                       // [n_ctx] scores, then e_t, then a_t
    uint16_t* vT = (uint16_t*)(sc + ((a.n_ctx + 3) & ~3));   // [2][D][TV] fp16 value tiles, dimension-major
    const float2* cs = a.rope_cs + (size_t)pos * half;
    const int last = max(nk - 2, 0);               // last cache row written by an earlier step

    // ---- requests first: waves 0 and 1 their q / k values, norm weights and rotation entries, then every thread its
    // key rows, then the loaders value tile 0. Loads complete in order, so with the key rows requested first the norm
    // below waited for them to come back from memory, while the q / k operands come from the previous kernel's
    // output (at head size 128 the early requests fit the 256 registers a 512-thread workgroup allows: 165) ----
    const uint64_t et = kExp2Tab[t & 31];          // (first: the waits for it and the gate input need nothing later)
    const float gin = row[Hq + 2 * kvd + h];
    const bool is_k = __builtin_amdgcn_readfirstlane(wv) == 1;   // (wave-uniform: the operand pointers stay scalar)
    float xq[DPL], wq[DPL], vq[DPL];
    float2 cq[DPL];
    auto load_qk = [&]() {
        const float* src = is_k ? row + Hq + g * D : row + h * D;
        const float* w = is_k ? a.k_norm : a.q_norm;
#pragma unroll
        for (int c = 0; c < DPL; c++) {
            const int e = min(lane + 64 * c, D - 1);   // (lanes past D re-read the last value; they use none)
            xq[c] = src[e];
            wq[c] = w[e];
            cq[c] = cs[e < half ? e : e - half];
            vq[c] = row[Hq + kvd + g * D + e];   // this position's v (cache row written by the k wave)
        }
    };
    if (wv < 2) load_qk();
    u32x4 ka[KW], kb[AHEAD2 ? KW : 1];
    {
        const int p0 = min(t, last), p1 = min(t + NT, last);
#pragma unroll
        for (int i = 0; i < KW; i++) ka[i] = ((const SH_GLOBAL u32x4*)(kc + (size_t)(s0 + p0) * D))[i];
        if (AHEAD2)
#pragma unroll
            for (int i = 0; i < KW; i++) kb[AHEAD2 ? i : 0] = ((const SH_GLOBAL u32x4*)(kc + (size_t)(s0 + p1) * D))[i];
    }
    // value staging: loader lt = t - 256 holds positions 8 * pb .. + 7 of a tile, dimensions 8 * kq .. + 7
    const int lt = t - 256, kq = lt & (KW - 1), pb = lt / KW;
    const bool loader = lt >= 0 && lt < NL;
    u32x4 vw[8];
    f32x4 vn0, vn1;                                // this position's v, dimensions 8 * kq .. + 7
    auto load_tile = [&](int j) {
#pragma unroll
        for (int r = 0; r < 8; r++) {
            const int p = min(j * TV + 8 * pb + r, last);
            vw[r] = ((const SH_GLOBAL u32x4*)(vc + (size_t)(s0 + p) * D))[kq];
        }
    };
    auto store_tile = [&](int j) {   // (this position's row replaced by its v)
        uint16_t* dst = vT + (size_t)(j & 1) * D * TV;
        const int rl = nk - 1 - (j * TV + 8 * pb);
        if (rl >= 0 && rl < 8) {
            const float f[8] = {vn0.x, vn0.y, vn0.z, vn0.w, vn1.x, vn1.y, vn1.z, vn1.w};
            unsigned wd[4];
#pragma unroll
            for (int e = 0; e < 4; e++) wd[e] = (unsigned)f2h(f[2 * e]) | ((unsigned)f2h(f[2 * e + 1]) << 16);
#pragma unroll
            for (int r = 0; r < 8; r++)
                if (r == rl) vw[r] = u32x4{wd[0], wd[1], wd[2], wd[3]};
        }
#pragma unroll
        for (int e = 0; e < 8; e++) {
            const unsigned sel = (e & 1) ? 0x07060302u : 0x05040100u;
            unsigned o4[4];
#pragma unroll
            for (int r = 0; r < 8; r += 2) {
                const unsigned lo = e >> 1 == 0 ? vw[r].x : e >> 1 == 1 ? vw[r].y : e >> 1 == 2 ? vw[r].z : vw[r].w;
                const unsigned hi = e >> 1 == 0 ? vw[r + 1].x : e >> 1 == 1 ? vw[r + 1].y : e >> 1 == 2 ? vw[r + 1].z : vw[r + 1].w;
                o4[r >> 1] = __builtin_amdgcn_perm(hi, lo, sel);
            }
            const int d = 8 * kq + e;
            *(u32x4*)(dst + (size_t)d * TV + 8 * (pb ^ vswz(d))) = u32x4{o4[0], o4[1], o4[2], o4[3]};
        }
    };

    if (loader) {   // tile 0 requested with the key rows (cache rows of earlier steps)
        load_tile(0);
        vn0 = ((const f32x4*)(row + Hq + kvd + g * D))[2 * kq];
        vn1 = ((const f32x4*)(row + Hq + kvd + g * D))[2 * kq + 1];
    }
    // ---- q (wave 0) and this position's k, v (wave 1): norm + NEOX rope (imi/core/seoul.cpp:19-28) ----
    if (wv < 2) {   // lane holds dimensions lane + 64 c; at D 128 a rope pair (i, i + 64) sits in one lane
        float* st = stg + wv * D;
        float x[DPL], n[DPL];
#pragma unroll
        for (int c = 0; c < DPL; c++) {
            const int e = lane + 64 * c;
            x[c] = e < D ? xq[c] : 0.0f;
            if (e < D) st[e] = x[c];
        }
        __builtin_amdgcn_wave_barrier();
        const float s = rms_scale_wave(st, D, a.eps);
#pragma unroll
        for (int c = 0; c < DPL; c++) n[c] = lane + 64 * c < D ? x[c] * s * wq[c] : 0.0f;
        const float sh = __shfl(n[0], lane < half ? lane + half : lane - half);
#pragma unroll
        for (int c = 0; c < DPL; c++) {
            const int e = lane + 64 * c;
            if (e < D) {
                const float other = DPL == 2 ? n[c ^ 1] : sh;
                const float2 cz = cq[c];
                const float r = e < half ? fmaf(n[c], cz.x, -(other * cz.y)) : fmaf(other, cz.y, n[c] * cz.x);
                if (is_k) {
                    const uint16_t kh = f2h(r);
                    k_s[e] = h2f(kh);
                    if (hh == 0) {
                        kc[(size_t)pos * D + e] = kh;
                        float v = vq[c];
                        asm volatile("" : "+v"(v));   // (keeps the conversion, and the wait for v, here)
                        vc[(size_t)pos * D + e] = f2h(v);
                    }
                } else {
                    q_s[e] = r;
                }
            }
        }
    }
    if (t < 32) etab[t] = et;
    __syncthreads();
    // ---- scores ----
    const float scale = 1.0f / sqrtf((float)D);
    for (int p = t; p < nk; p += NT) {
        if (D > 64 && p != t) {   // D 128: this pass's row requested here (no prefetch registers to spare)
#pragma unroll
            for (int i = 0; i < KW; i++) ka[i] = ((const SH_GLOBAL u32x4*)(kc + (size_t)(s0 + min(p, last)) * D))[i];
        }
        if (D > 64) {   // dot_h's 8 chains over columns i % 8, a word (8 columns) at a time
            // (q read from LDS in the loop, and the position's own key row (from LDS) and the cache rows (converted
            // from the registers) in two loops: with one loop holding both, all 128 key values were converted ahead of
            // the products and the kernel went past 256 registers into scratch)
            asm volatile("" ::: "memory");
            float acc[8];
#pragma unroll
            for (int l = 0; l < 8; l++) acc[l] = 0.0f;
            if (p == nk - 1) {
#pragma unroll
                for (int i = 0; i < KW; i++) {
                    const f32x4 qa = *(const f32x4*)(q_s + 8 * i), qb = *(const f32x4*)(q_s + 8 * i + 4);
                    const f32x4 ka4 = *(const f32x4*)(k_s + 8 * i), kb4 = *(const f32x4*)(k_s + 8 * i + 4);
                    const float qv[8] = {qa.x, qa.y, qa.z, qa.w, qb.x, qb.y, qb.z, qb.w};
                    const float kv[8] = {ka4.x, ka4.y, ka4.z, ka4.w, kb4.x, kb4.y, kb4.z, kb4.w};
#pragma unroll
                    for (int l = 0; l < 8; l++) acc[l] = fmaf(qv[l], kv[l], acc[l]);
                }
            } else {
#pragma unroll
                for (int i = 0; i < KW; i++) {
                    const f32x4 qa = *(const f32x4*)(q_s + 8 * i), qb = *(const f32x4*)(q_s + 8 * i + 4);
                    const float qv[8] = {qa.x, qa.y, qa.z, qa.w, qb.x, qb.y, qb.z, qb.w};
                    const unsigned w4[4] = {ka[i].x, ka[i].y, ka[i].z, ka[i].w};
                    float kv[8];
#pragma unroll
                    for (int e = 0; e < 8; e++) kv[e] = h2f((uint16_t)((w4[e >> 1] >> (16 * (e & 1))) & 0xFFFFu));
#pragma unroll
                    for (int l = 0; l < 8; l++) acc[l] = fmaf(qv[l], kv[l], acc[l]);
                }
            }
            sc[p] = (((acc[0] + acc[4]) + (acc[2] + acc[6])) + ((acc[1] + acc[5]) + (acc[3] + acc[7]))) * scale;
            continue;
        }
        u32x4 kn[KW];
        const int pn = min(p + (AHEAD2 ? 2 : 1) * NT, last);
#pragma unroll
        for (int i = 0; i < KW; i++) kn[i] = ((const SH_GLOBAL u32x4*)(kc + (size_t)(s0 + pn) * D))[i];
        float kf[D];
        if (p == nk - 1) {
#pragma unroll
            for (int i = 0; i < D; i++) kf[i] = k_s[i];
        } else {
#pragma unroll
            for (int i = 0; i < KW; i++) {
                const unsigned w4[4] = {ka[i].x, ka[i].y, ka[i].z, ka[i].w};
#pragma unroll
                for (int e = 0; e < 8; e++) kf[8 * i + e] = h2f((uint16_t)((w4[e >> 1] >> (16 * (e & 1))) & 0xFFFFu));
            }
        }
        sc[p] = dot_h8<D>(q_s, kf) * scale;
        if (AHEAD2) {
#pragma unroll
            for (int i = 0; i < KW; i++) { ka[i] = kb[AHEAD2 ? i : 0]; kb[AHEAD2 ? i : 0] = kn[i]; }
        } else {
#pragma unroll
            for (int i = 0; i < KW; i++) ka[i] = kn[i];
        }
    }
    if (loader) {   // tile 0 to LDS, tile 1 requested (waves 4-7 hold no scores below 256 positions)
        store_tile(0);
        if (ntile > 1) load_tile(1);
    }
    __syncthreads();
    // ---- softmax ----
    float mx = -INFINITY;
    for (int p = t; p < nk; p += NT) mx = fmaxf(mx, sc[p]);
    mx = wave_max_dpp(mx);
    if (lane == 0) red[wv] = mx;
    __syncthreads();
    mx = red[0];
#pragma unroll
    for (int w = 1; w < NT / 64; w++) mx = fmaxf(mx, red[w]);
    double part = 0.0;
    int lowb = 1 << 20;
    for (int p = t; p < nk; p += NT) {
        const float e = expf_glibc_t(sc[p] - mx, etab);
        sc[p] = e;
        part += (double)e;
        lowb = min(lowb, low_bit_exp(e));
    }
    // wave totals: DPP levels within each 16-lane row, then the four rows (the tree's order is free: its total is
    // used only when every partial sum is exact)
    part += dppd<DPP_XOR1>(part);
    lowb = min(lowb, dppi<DPP_XOR1>(lowb));
    part += dppd<DPP_XOR2>(part);
    lowb = min(lowb, dppi<DPP_XOR2>(lowb));
    part += dppd<DPP_MIRROR8>(part);
    lowb = min(lowb, dppi<DPP_MIRROR8>(lowb));
    part += dppd<DPP_MIRROR16>(part);
    lowb = min(lowb, dppi<DPP_MIRROR16>(lowb));
    // (the lane reads stay outside the lane-0 branch: inside it the last level's adds may be moved into the branch
    // too, leaving lanes 16, 32 and 48 with their 8-lane values)
    const double wsum = (readlane_d(part, 0) + readlane_d(part, 16)) + (readlane_d(part, 32) + readlane_d(part, 48));
    const int wlow = min(min(__builtin_amdgcn_readlane(lowb, 0), __builtin_amdgcn_readlane(lowb, 16)),
                         min(__builtin_amdgcn_readlane(lowb, 32), __builtin_amdgcn_readlane(lowb, 48)));
    if (lane == 0) { red_d[wv] = wsum; red_i[wv] = wlow; }
    __syncthreads();
    // 1 / sum on wave 0 only, which runs the value chains: no barrier after it (every lane computes the same value);
    // the head gate there too, ahead of the chains, whose dependent steps leave room for its instructions
    float inv = 0.0f, gate = 0.0f;
    if (wv == 0) {
        gate = 1.0f / (1.0f + expf_glibc_t(-gin, etab));
        double tot = 0.0;
        int lb = 1 << 20;
#pragma unroll
        for (int w = 0; w < NT / 64; w++) { tot += red_d[w]; lb = min(lb, red_i[w]); }
        int ex;
        (void)frexp(tot, &ex);   // tot = f * 2^ex, f in [0.5, 1): floor(log2(tot)) = ex - 1
        if (lb < ex - 1 - 51) {  // some e_t below the exact unit: add in position order
            double sum = 0.0;
            int p = 0;
            for (; p + 8 <= nk; p += 8) {
                float v[8];
#pragma unroll
                for (int u = 0; u < 8; u++) v[u] = sc[p + u];
#pragma unroll
                for (int u = 0; u < 8; u++) sum += (double)v[u];
            }
            for (; p < nk; p++) sum += (double)sc[p];
            tot = sum;
        }
        inv = (float)(1.0 / tot);
    }
    // ---- o = sum_t fma(a_t, V_t, o), lane i of wave 0; tiles double-buffered through LDS ----
    float o[DPL];
#pragma unroll
    for (int c = 0; c < DPL; c++) o[c] = 0.0f;
    for (int j = 0; j < ntile; j++) {
        if (wv == 0 && lane < D) {   // dimension lane + 64 c's chain (two independent chains per lane at D 128)
            const int q0 = j * TV, nt = min(TV, nk - q0);
            const float* ar = sc + q0;
            int fz[DPL];
            const uint16_t* vr[DPL];
#pragma unroll
            for (int c = 0; c < DPL; c++) {
                fz[c] = vswz(lane + 64 * c);
                vr[c] = vT + (size_t)(j & 1) * D * TV + (size_t)(lane + 64 * c) * TV;
            }
            int p = 0;
            // 32 positions at a time, the next group's weights and values read from LDS before this group's chain
            // runs (register double buffer, static indices; the last group re-reads itself, unused)
            auto load32 = [&](int p32, float (&aa)[32], unsigned (&vv)[DPL][16]) {
#pragma unroll
                for (int q = 0; q < 8; q++) {
                    const f32x4 x = *(const f32x4*)(ar + p32 + 4 * q);
                    aa[4 * q] = x.x * inv; aa[4 * q + 1] = x.y * inv; aa[4 * q + 2] = x.z * inv; aa[4 * q + 3] = x.w * inv;
                }
#pragma unroll
                for (int c = 0; c < DPL; c++)
#pragma unroll
                    for (int q = 0; q < 4; q++) {
                        const u32x4 w = *(const u32x4*)(vr[c] + 8 * (((p32 >> 3) + q) ^ fz[c]));
                        vv[c][4 * q] = w.x; vv[c][4 * q + 1] = w.y; vv[c][4 * q + 2] = w.z; vv[c][4 * q + 3] = w.w;
                    }
            };
            auto chain32 = [&](const float (&aa)[32], const unsigned (&vv)[DPL][16]) {
#pragma unroll
                for (int c = 0; c < DPL; c++)
#pragma unroll
                    for (int u = 0; u < 32; u++)
                        o[c] = fmaf(aa[u], h2f((uint16_t)((vv[c][u >> 1] >> (16 * (u & 1))) & 0xFFFFu)), o[c]);
            };
            if (nt >= 32) {
                float a0[32], a1[32];
                unsigned v0[DPL][16], v1[DPL][16];
                load32(0, a0, v0);
                for (;;) {
                    const bool more = p + 64 <= nt;
                    load32(more ? p + 32 : p, a1, v1);
                    chain32(a0, v0);
                    p += 32;
                    if (!more) break;
                    const bool more2 = p + 64 <= nt;
                    load32(more2 ? p + 32 : p, a0, v0);
                    chain32(a1, v1);
                    p += 32;
                    if (!more2) break;
                }
            }
            for (; p + 8 <= nt; p += 8) {
                const f32x4 a0 = *(const f32x4*)(ar + p), a1 = *(const f32x4*)(ar + p + 4);
                const float av[8] = {a0.x * inv, a0.y * inv, a0.z * inv, a0.w * inv,
                                     a1.x * inv, a1.y * inv, a1.z * inv, a1.w * inv};
#pragma unroll
                for (int c = 0; c < DPL; c++) {
                    const u32x4 w = *(const u32x4*)(vr[c] + 8 * ((p >> 3) ^ fz[c]));
                    const unsigned ws[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
                    for (int u = 0; u < 8; u++) o[c] = fmaf(av[u], h2f((uint16_t)((ws[u >> 1] >> (16 * (u & 1))) & 0xFFFFu)), o[c]);
                }
            }
            if (p < nt) {
#pragma unroll
                for (int c = 0; c < DPL; c++) {
                    const u32x4 w = *(const u32x4*)(vr[c] + 8 * ((p >> 3) ^ fz[c]));
                    const unsigned ws[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
                    for (int u = 0; u < 8; u++)
                        if (p + u < nt) o[c] = fmaf(ar[p + u] * inv, h2f((uint16_t)((ws[u >> 1] >> (16 * (u & 1))) & 0xFFFFu)), o[c]);
                }
            }
        }
        if (loader && j + 1 < ntile) {
            store_tile(j + 1);
            if (j + 2 < ntile) load_tile(j + 2);
        }
        __syncthreads();
    }
    if (wv == 0 && lane < D) {
#pragma unroll
        for (int c = 0; c < DPL; c++)
            if (lane + 64 * c < D) a.att[(size_t)m * Hq + h * D + lane + 64 * c] = o[c] * gate;
    }
}

static size_t attn_head_lds(int D, int n_ctx) {
    const size_t tv = D > 64 ? attn_detail::tile_positions<128>() : attn_detail::tile_positions<64>();
    return sizeof(float) * (4 * (size_t)D + 32 + 16 + 8 + 64 + (((size_t)n_ctx + 3) & ~(size_t)3)) + 2 * (size_t)D * tv * sizeof(uint16_t);
}

// the longest context the decode attention holds: its score row (one float per position) and two value tiles share
// the workgroup's 160 KB of LDS
int attn_max_ctx(int grp, int D) {
    (void)grp;
    int lo = 0, hi = 1 << 20;
    while (lo < hi) {
        const int mid = (lo + hi + 1) / 2;
        if (attn_head_lds(D, mid) <= 160 * 1024) lo = mid;
        else hi = mid - 1;
    }
    return lo;
}

// ---------------------------------------------------------------- end of step
// Hidden state when no word scores were computed (x += norm(y) * w_post; hidden = norm(x) * w_out, in the CPU's
// op order), argmax over the word-score partials (first index of the maximum), position advance and the
// device-side greedy bookkeeping. One block of 256 threads; the norms run on wave 0.
template <int M>
__global__ __launch_bounds__(256) void k_final(final_args a) {
    extern __shared__ float lds[];
    __shared__ float red_v[256];
    __shared__ int red_i[256];
    const int tid = threadIdx.x, E = a.E;
    float* l_x = lds;   // [E]
    // the parameter-block words thread 0 updates at the end, requested before everything else, one per lane of wave
    // 0 (lanes 0-7: token, pos, best, n_done, greedy; 8-11: the two out_tok pointers) and taken by lane reads after
    // the pick: read there, each was one more memory round trip in a row (this kernel is their only writer)
    static_assert(offsetof(step_params, pos) == 8 && offsetof(step_params, n_done) == 24 &&
                  offsetof(step_params, greedy) == 28 && offsetof(step_params, out_tok) == 80, "step_params layout");
    SH_GLOBAL step_params* const P = global_ptr(a.P);
    const int pv = ((const SH_GLOBAL int*)P)[tid < 8 ? tid : tid < 12 ? 12 + tid : 0];
    // every conversation's first partial and score 0 requested before the picks too (at two conversations the
    // second's loads otherwise went out after the first's pick); score 0 by a load on every path (without scores it
    // reads a partial, unused: a conditional load had its NaN test, and a wait for it, ahead of the partials)
    float pv0[M], l0v[M];
    int pi0[M];
    if (a.part_v) {
        const int k0 = tid < a.n_part ? tid : a.n_part - 1;
#pragma unroll
        for (int m = 0; m < M; m++) {
            pv0[m] = a.part_v[m * a.n_part + k0];
            pi0[m] = a.part_i[m * a.n_part + k0];
            l0v[m] = (a.logits ? a.logits : a.part_v)[a.logits ? (size_t)m * a.ld_logits : 0];
        }
    }
    int bests[M];
#pragma unroll
    for (int m = 0; m < M; m++) {
        if (a.hidden_out && a.x_in) {
            if (a.y_in) {
                for (int i = tid; i < E; i += 256) l_x[i] = a.y_in[m * E + i];
                __syncthreads();
                if (tid < 64) red_v[tid] = rms_scale_wave(l_x, E, a.eps);
                __syncthreads();
                const float sc1 = red_v[0];
                __syncthreads();
                for (int i = tid; i < E; i += 256) l_x[i] = fmaf(a.y_in[m * E + i] * sc1, a.w_post[i], a.x_in[m * E + i]);
            } else {
                for (int i = tid; i < E; i += 256) l_x[i] = a.x_in[m * E + i];
            }
            __syncthreads();
            if (tid < 64) red_v[tid] = rms_scale_wave(l_x, E, a.eps);
            __syncthreads();
            const float sc2 = red_v[0];
            for (int i = tid; i < E; i += 256) a.hidden_out[m * E + i] = l_x[i] * sc2 * a.w_out[i];
            __syncthreads();
        }
    }
    // the picks of every conversation at once (their shuffle trees interleave; one LDS exchange and barrier for all)
#pragma unroll
    for (int m = 0; m < M; m++) bests[m] = -1;
    if (a.part_v) {
        float v[M];
        int bi[M];
#pragma unroll
        for (int m = 0; m < M; m++) {
            v[m] = tid < a.n_part ? pv0[m] : -INFINITY;
            bi[m] = tid < a.n_part ? pi0[m] : 0x7fffffff;
            for (int k = tid + 256; k < a.n_part; k += 256) {
                const float ov = a.part_v[m * a.n_part + k];
                const int oi = a.part_i[m * a.n_part + k];
                if (ov > v[m] || (ov == v[m] && oi < bi[m])) { v[m] = ov; bi[m] = oi; }
            }
        }
        // (greater score, or equal score and lower row, wins: a total order on the partials, none of them NaN, so
        // any reduction order picks the same row) by shuffles within each wave, then the 4 waves' picks
#pragma unroll
        for (int o = 32; o > 0; o >>= 1)
#pragma unroll
            for (int m = 0; m < M; m++) {
                const float ov = __shfl_xor(v[m], o);
                const int oi = __shfl_xor(bi[m], o);
                if (ov > v[m] || (ov == v[m] && oi < bi[m])) { v[m] = ov; bi[m] = oi; }
            }
        if ((tid & 63) == 0)
#pragma unroll
            for (int m = 0; m < M; m++) { red_v[4 * m + (tid >> 6)] = v[m]; red_i[4 * m + (tid >> 6)] = bi[m]; }
        __syncthreads();
#pragma unroll
        for (int m = 0; m < M; m++) {
            float bv = red_v[4 * m];
            int bj = red_i[4 * m];
#pragma unroll
            for (int w = 1; w < 4; w++)
                if (red_v[4 * m + w] > bv || (red_v[4 * m + w] == bv && red_i[4 * m + w] < bj)) { bv = red_v[4 * m + w]; bj = red_i[4 * m + w]; }
            // imi's loop (imi/core/hear.cpp:67-68): best = 0, then v replaces it only if logits[v] > logits[best].
            // The partials give the first maximum over the scores that are not NaN; imi keeps 0 when score 0 is NaN
            // (nothing compares greater than it) and when every score is NaN (the partials then hold no row)
            int best = bj;
            if (best < 0 || best >= a.ld_logits || (a.logits && isnan(l0v[m]))) best = 0;
            bests[m] = best;
        }
    }
    // (the lane reads stay outside the thread-0 branch, so the loads above run on all of wave 0's lanes)
    const int n_done = __builtin_amdgcn_readlane(pv, 6), greedy = __builtin_amdgcn_readlane(pv, 7);
    int pos_m[M];
    int32_t* out_m[M];
#pragma unroll
    for (int m = 0; m < M; m++) {
        pos_m[m] = __builtin_amdgcn_readlane(pv, 2 + m);
        out_m[m] = (int32_t*)(((unsigned long long)(unsigned)__builtin_amdgcn_readlane(pv, 9 + 2 * m) << 32) |
                              (unsigned)__builtin_amdgcn_readlane(pv, 8 + 2 * m));
    }
    if (tid == 0) {
#pragma unroll
        for (int m = 0; m < M; m++) {
            P->best[m] = bests[m];
            if (a.advance) {
                if (greedy && out_m[m]) global_ptr(out_m[m])[n_done] = bests[m];
                if (greedy) P->token[m] = bests[m];
                P->pos[m] = pos_m[m] + 1;
            }
        }
        if (a.advance) P->n_done = n_done + 1;
    }
}

// e^x of n floats with the kernels' exponential (for checks against the C library)
__global__ void k_expf(const float* x, float* y, long long n) {
    const long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) y[i] = expf_glibc(x[i]);
}

// ---------------------------------------------------------------- dequantized rows
__global__ __launch_bounds__(64) void k_q4_rows(q4dev T, const int32_t* ids, float* out) {
    const int i = blockIdx.x, row = ids[i];
    for (int blk = threadIdx.x; blk < T.nb; blk += 64) {
        float v[32];
        q4_dequant_block(T, row, blk, v);
        store32(out + (size_t)i * T.cols + 32 * blk, v);
    }
}

// ---------------------------------------------------------------- launchers
// with t0/t1 set, the launch records them around the kernel itself (hipExtLaunchKernelGGL), which times the
// kernel's own duration without the dispatch gap in front of it
#define SH_GEMV_CASE(M_, NBL_, PRO_, EPI_, UG_)                                                                  \
    if (M == M_ && nbl == NBL_ && pro == PRO_ && epi == EPI_ && ug == UG_) {                                     \
        const size_t lds = gemv_lds(M_, UG_, a.W.nb, a.E, PRO_ == PRO_EMBED_NORM || PRO_ == PRO_RESID_NORM);     \
        if (lds > 64 * 1024) return hipErrorInvalidValue;                                                        \
        if (t0) hipExtLaunchKernelGGL((k_gemv<M_, NBL_, PRO_, EPI_, UG_>), dim3(grid), dim3(64), lds, s, t0, t1, 0, a); \
        else hipLaunchKernelGGL((k_gemv<M_, NBL_, PRO_, EPI_, UG_>), dim3(grid), dim3(64), lds, s, a);           \
        return hipGetLastError();                                                                                \
    }

// tables behind the post-norm residual that k_gemv_norm takes (E a multiple of 128 up to 2048, the table's input E)
static bool norm_kernel_takes(int M, int pro, const gemv_args& a, int ug) {
    const bool resid = pro == PRO_RESID_NORM && a.x_in && a.y_in && a.w_post;
    const bool embed = pro == PRO_EMBED_NORM && (a.emb.codes || a.emb6.codes) && a.embd;
    return (resid || embed) && (M == 1 || M == 2) && (a.E == 256 || a.E == 512 || a.E == 1024 || a.E == 2048) && a.W.nb * 32 == a.E &&
           a.W.cols == a.E && a.W.rows % (8 * ug) == 0;
}

int gemv_logits_grid(int M, int pro, const gemv_args& a, int max_grid) {
    if (norm_kernel_takes(M, pro, a, 1)) return 256;   // k_gemv_norm: one workgroup per compute unit, chunks looped
    return a.units < max_grid ? a.units : max_grid;
}

hipError_t launch_scores_q6k(int M, int grid, const gemv_args& a, hipStream_t s, hipEvent_t t0, hipEvent_t t1) {
    const bool e_ok = a.E == 256 || a.E == 512 || a.E == 1024 || a.E == 2048;
    if ((M != 1 && M != 2) || !e_ok || !a.W6.codes || a.W6.cols != a.E || a.W6.nbk * 256 != a.E || grid < 1 || !a.part_v ||
        !a.part_i || (!a.src && (!a.x_in || !a.w_pre || (a.y_in && !a.w_post))))
        return hipErrorInvalidValue;
    const void* fn = M == 2 ? (const void*)k_scores_q6k<2> : (const void*)k_scores_q6k<1>;
    const size_t lds = scores_q6k_lds(M, a.E);
    if (lds > 64 * 1024) {
        const hipError_t e = hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
        if (e != hipSuccess) return e;
    }
    gemv_args b = a;
    void* args[] = {&b};
    return hipExtLaunchKernel(fn, dim3(grid), dim3(512), args, lds, s, t0, t1, 0);
}

bool swiglu_cut_takes(int M, const gemv_args& gate_up, const gemv_args& down) {
    return (M == 1 || M == 2) && norm_kernel_takes(M, PRO_RESID_NORM, gate_up, 2) && !gate_up.W.mins && gate_up.units % 4 == 0 &&
           gate_up.units >= 4 && !down.W.mins && down.W.rows % 8 == 0 &&
           (down.W.nb == 64 || down.W.nb == 128 || down.W.nb == 256 || nb_runtime256(down.W.nb)) && down.W.cols == 8 * gate_up.units;
}

hipError_t launch_gemv(int M, int pro, int epi, int grid, const gemv_args& a, hipStream_t s, hipEvent_t t0, hipEvent_t t1) {
    const int nbl = (a.W.nb + 63) / 64;
    const int ug = epi == EPI_SWIGLU ? 2 : epi == EPI_CONV ? 3 : 1;
    if (norm_kernel_takes(M, pro, a, ug) && (epi != EPI_CONV || a.d_conv <= 8)) {
        gemv_args b = a;
        // units per chunk: 8 groups for the word scores (looped), else enough that one round of workgroups (one
        // per compute unit: the register use allows one 512-thread workgroup per unit) covers the table
        const int cap = 8 / ug, want = (a.units + 255) / 256;
        b.upw = a.upw > 0 ? a.upw : epi == EPI_LOGITS ? 8 : (want < 1 ? 1 : want > cap ? cap : want);
        // the cut epilogue needs every chunk to be one whole 32-channel block
        if (a.outq && (epi != EPI_SWIGLU || b.upw != 4 || a.units % 4 != 0 || a.W.mins)) return hipErrorInvalidValue;
        const int nchunk = (a.units + b.upw - 1) / b.upw;
        const void* fn = nullptr;
        const bool hm = a.W.mins != nullptr;
        if (pro == PRO_EMBED_NORM) {   // layer 0: the embedding row in the prologue
            if (epi != EPI_STORE && epi != EPI_CONV) return hipErrorInvalidValue;
#define SH_EMB_FN(M_, EPI_, UG_) if (M == M_ && epi == EPI_) fn = hm ? (const void*)k_gemv_norm<M_, EPI_, UG_, true, true> : (const void*)k_gemv_norm<M_, EPI_, UG_, false, true>;
            SH_EMB_FN(1, EPI_STORE, 1) SH_EMB_FN(1, EPI_CONV, 3) SH_EMB_FN(2, EPI_STORE, 1) SH_EMB_FN(2, EPI_CONV, 3)
#undef SH_EMB_FN
        } else {
            // the rows per thread the chunk gives (as the kernel derives them); the shapes the decode step runs take
            // a kernel with them fixed at compile time (row and scale indices then static, no per-row branches)
            const int np = b.upw * ug * a.W.nb, rptv = np <= 64 ? 1 : np <= 128 ? 2 : np <= 256 ? 4 : 8;
#define SH_NORM_R(M_, EPI_, UG_, R_) if (!fn && !hm && M == M_ && epi == EPI_ && rptv == R_ && np <= 512) fn = (const void*)k_gemv_norm<M_, EPI_, UG_, false, false, R_>;
            SH_NORM_R(1, EPI_STORE, 1, 2) SH_NORM_R(1, EPI_STORE, 1, 8) SH_NORM_R(1, EPI_SWIGLU, 2, 8) SH_NORM_R(1, EPI_CONV, 3, 4)
            SH_NORM_R(1, EPI_CONV, 3, 8) SH_NORM_R(1, EPI_LOGITS, 1, 8)
            SH_NORM_R(2, EPI_STORE, 1, 2) SH_NORM_R(2, EPI_STORE, 1, 8) SH_NORM_R(2, EPI_SWIGLU, 2, 8) SH_NORM_R(2, EPI_CONV, 3, 4)
            SH_NORM_R(2, EPI_CONV, 3, 8) SH_NORM_R(2, EPI_LOGITS, 1, 8)
#undef SH_NORM_R
#define SH_NORM_FN(M_, EPI_, UG_) if (!fn && M == M_ && epi == EPI_) fn = hm ? (const void*)k_gemv_norm<M_, EPI_, UG_, true> : (const void*)k_gemv_norm<M_, EPI_, UG_>;
            SH_NORM_FN(1, EPI_STORE, 1) SH_NORM_FN(1, EPI_SWIGLU, 2) SH_NORM_FN(1, EPI_CONV, 3) SH_NORM_FN(1, EPI_LOGITS, 1)
            SH_NORM_FN(2, EPI_STORE, 1) SH_NORM_FN(2, EPI_SWIGLU, 2) SH_NORM_FN(2, EPI_CONV, 3) SH_NORM_FN(2, EPI_LOGITS, 1)
#undef SH_NORM_FN
        }
        if (!fn) return hipErrorInvalidValue;
        const size_t lds = gemv_norm_lds(M, a.E, a.W.nb, b.upw * ug, epi == EPI_LOGITS ? (nchunk + grid - 1) / grid : 0);
        if (lds > 160 * 1024) return hipErrorInvalidValue;
        if (lds > 64 * 1024) {
            const hipError_t e = hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
            if (e != hipSuccess) return e;
        }
        void* args[] = {&b};
        const dim3 gr(epi == EPI_LOGITS ? grid : nchunk), bl(512);
        if (t0) return hipExtLaunchKernel(fn, gr, bl, args, lds, s, t0, t1, 0);
        return hipLaunchKernel(fn, gr, bl, args, lds, s);
    }
    // the plain tables (input cut, rows stored): one workgroup per 8-row group, the grid is the group count
    const int nb = a.W.nb;
    if (pro == PRO_PRECUT) {   // the input arrives cut: Q4_0 tables of 64, 128 or 256 blocks
        if (epi != EPI_STORE || a.W.mins || a.W.rows % 8 != 0 || !a.src_q || !a.src_d || !a.src_s || (M != 1 && M != 2))
            return hipErrorInvalidValue;
        const void* fn = nullptr;
#define SH_PRE_FN(M_, NB_) if (M == M_ && nb == NB_) fn = (const void*)k_gemv_cut<M_, false, NB_, false, true>;
        SH_PRE_FN(1, 64) SH_PRE_FN(1, 128) SH_PRE_FN(1, 256) SH_PRE_FN(2, 64) SH_PRE_FN(2, 128) SH_PRE_FN(2, 256)
#undef SH_PRE_FN
        if (nb_runtime256(nb)) fn = M == 1 ? (const void*)k_gemv_cut<1, false, 256, false, true, true> : (const void*)k_gemv_cut<2, false, 256, false, true, true>;
        if (!fn) return hipErrorInvalidValue;
        void* args[] = {const_cast<gemv_args*>(&a)};
        const dim3 gr(a.W.rows / 8), bl(256);
        const size_t lds = gemv_cut_lds(M, nb_runtime256(nb) ? 256 : nb);
        if (t0) return hipExtLaunchKernel(fn, gr, bl, args, lds, s, t0, t1, 0);
        return hipLaunchKernel(fn, gr, bl, args, lds, s);
    }
    if (epi == EPI_STORE && (pro == PRO_CUT || pro == PRO_CUT_HALF_AWAY) &&
        (nb == 64 || nb == 128 || nb == 256 || (nb_runtime256(nb) && pro == PRO_CUT && !a.W.mins)) &&
        a.W.rows % 8 == 0 && (M == 1 || (M == 2 && pro == PRO_CUT))) {
        const bool half = pro == PRO_CUT_HALF_AWAY, hm = a.W.mins != nullptr;
        if (half && hm) return hipErrorInvalidValue;   // q4x8's cut is for Q4_0 tables only
        const void* fn = nullptr;
        if (nb_runtime256(nb) && !half && !hm)   // 240-style widths: the 256-block body with the runtime count
            fn = M == 1 ? (const void*)k_gemv_cut<1, false, 256, false, false, true> : (const void*)k_gemv_cut<2, false, 256, false, false, true>;
#define SH_CUT_FN(M_, H_, NB_) if (M == M_ && half == H_ && nb == NB_) fn = (const void*)k_gemv_cut<M_, H_, NB_>;
#define SH_CUT_FN1(M_, NB_) if (M == M_ && nb == NB_) fn = (const void*)k_gemv_cut<M_, false, NB_, true>;
        if (hm) {
            SH_CUT_FN1(1, 64) SH_CUT_FN1(1, 128) SH_CUT_FN1(1, 256) SH_CUT_FN1(2, 64) SH_CUT_FN1(2, 128) SH_CUT_FN1(2, 256)
        } else {
            SH_CUT_FN(1, false, 64) SH_CUT_FN(1, false, 128) SH_CUT_FN(1, false, 256)
            SH_CUT_FN(1, true, 64) SH_CUT_FN(1, true, 128) SH_CUT_FN(1, true, 256)
            SH_CUT_FN(2, false, 64) SH_CUT_FN(2, false, 128) SH_CUT_FN(2, false, 256)
        }
#undef SH_CUT_FN
#undef SH_CUT_FN1
        void* args[] = {const_cast<gemv_args*>(&a)};
        const dim3 gr(a.W.rows / 8), bl(256);
        const size_t lds = gemv_cut_lds(M, nb_runtime256(nb) ? 256 : nb);
        if (t0) return hipExtLaunchKernel(fn, gr, bl, args, lds, s, t0, t1, 0);
        return hipLaunchKernel(fn, gr, bl, args, lds, s);
    }
    SH_GEMV_CASE(1, 1, PRO_CUT, EPI_STORE, 1) SH_GEMV_CASE(2, 1, PRO_CUT, EPI_STORE, 1)
    SH_GEMV_CASE(1, 2, PRO_CUT, EPI_STORE, 1) SH_GEMV_CASE(2, 2, PRO_CUT, EPI_STORE, 1)
    SH_GEMV_CASE(1, 3, PRO_CUT, EPI_STORE, 1) SH_GEMV_CASE(2, 3, PRO_CUT, EPI_STORE, 1)
    SH_GEMV_CASE(1, 4, PRO_CUT, EPI_STORE, 1) SH_GEMV_CASE(2, 4, PRO_CUT, EPI_STORE, 1)
    SH_GEMV_CASE(1, 1, PRO_CUT_HALF_AWAY, EPI_STORE, 1) SH_GEMV_CASE(1, 2, PRO_CUT_HALF_AWAY, EPI_STORE, 1)
    SH_GEMV_CASE(1, 3, PRO_CUT_HALF_AWAY, EPI_STORE, 1) SH_GEMV_CASE(1, 4, PRO_CUT_HALF_AWAY, EPI_STORE, 1)
    SH_GEMV_CASE(1, 1, PRO_EMBED_NORM, EPI_STORE, 1) SH_GEMV_CASE(2, 1, PRO_EMBED_NORM, EPI_STORE, 1)
    SH_GEMV_CASE(1, 1, PRO_EMBED_NORM, EPI_CONV, 3) SH_GEMV_CASE(2, 1, PRO_EMBED_NORM, EPI_CONV, 3)
    SH_GEMV_CASE(1, 1, PRO_RESID_NORM, EPI_STORE, 1) SH_GEMV_CASE(2, 1, PRO_RESID_NORM, EPI_STORE, 1)
    SH_GEMV_CASE(1, 1, PRO_RESID_NORM, EPI_CONV, 3) SH_GEMV_CASE(2, 1, PRO_RESID_NORM, EPI_CONV, 3)
    SH_GEMV_CASE(1, 1, PRO_RESID_NORM, EPI_SWIGLU, 2) SH_GEMV_CASE(2, 1, PRO_RESID_NORM, EPI_SWIGLU, 2)
    SH_GEMV_CASE(1, 1, PRO_RESID_NORM, EPI_LOGITS, 1) SH_GEMV_CASE(2, 1, PRO_RESID_NORM, EPI_LOGITS, 1)
    SH_GEMV_CASE(1, 1, PRO_CUT, EPI_LOGITS, 1)
    return hipErrorInvalidValue;
}

hipError_t launch_gemv_group(int M, bool half, const gemv_group_args& g, hipStream_t s, hipEvent_t t0, hipEvent_t t1) {
    if (g.n < 1 || g.n > GEMV_GROUP_MAX || M < 1 || M > 2 || (half && M != 1)) return hipErrorInvalidValue;
    if (g.start[0] != 0) return hipErrorInvalidValue;
    size_t lds = 0;
    for (int i = 0; i < g.n; i++) {   // Q4_0 tables of 64, 128 or 256 blocks per row, whole groups of 8 rows
        const int nb = g.W[i].nb;
        if ((nb != 64 && nb != 128 && nb != 256) || g.W[i].mins || g.W[i].rows % 8 ||
            g.W[i].rows < 8 || g.start[i + 1] - g.start[i] != g.W[i].rows / 8 || !g.src[i] || !g.out[i])
            return hipErrorInvalidValue;
        lds = std::max(lds, gemv_cut_lds(M, nb));
    }
    int nbf = g.W[0].nb;
    for (int i = 1; i < g.n; i++)
        if (g.W[i].nb != nbf) nbf = 0;
    const void* fn = nullptr;
#define SH_GRP(M_, H_)                                                                                             \
    if (M == M_ && half == H_)                                                                                     \
        fn = nbf == 64 ? (const void*)k_gemv_cut_group<M_, H_, 64> : nbf == 128 ? (const void*)k_gemv_cut_group<M_, H_, 128> \
           : nbf == 256 ? (const void*)k_gemv_cut_group<M_, H_, 256> : (const void*)k_gemv_cut_group<M_, H_, 0>;
    SH_GRP(1, false) SH_GRP(1, true) SH_GRP(2, false)
#undef SH_GRP
    if (!fn) return hipErrorInvalidValue;
    void* args[] = {const_cast<gemv_group_args*>(&g)};
    const dim3 gr(g.start[g.n]), bl(256);
    if (t0) return hipExtLaunchKernel(fn, gr, bl, args, lds, s, t0, t1, 0);
    return hipLaunchKernel(fn, gr, bl, args, lds, s);
}

hipError_t launch_q4_rows(const q4dev& T, const int32_t* ids, int n, float* out, hipStream_t s) {
    hipLaunchKernelGGL(k_q4_rows, dim3(n), dim3(64), 0, s, T, ids, out);
    return hipGetLastError();
}

hipError_t launch_attn(int M, const attn_args& a, hipStream_t s) {
    const int grp = a.n_head / a.n_kv;
    const size_t lds = sizeof(float) * ((size_t)grp * a.D + (size_t)grp * a.n_ctx + 5 * (size_t)a.D + (size_t)grp);
    if (lds > 160 * 1024) return hipErrorInvalidValue;
    {   // one block per query head
        const size_t lds2 = attn_head_lds(a.D, a.n_ctx);
        const void* fh = a.D == 128 ? (const void*)k_attn_head<128> : a.D == 64 ? (const void*)k_attn_head<64>
                       : a.D == 32 ? (const void*)k_attn_head<32> : nullptr;
        if (fh && lds2 <= 160 * 1024) {
            if (lds2 > 64 * 1024) {
                const hipError_t e = hipFuncSetAttribute(fh, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds2);
                if (e != hipSuccess) return e;
            }
            attn_args b = a;
            void* args[] = {&b};
            return hipLaunchKernel(fh, dim3(a.n_head, M), dim3(attn_detail::NT), args, lds2, s);
        }
    }
    const void* fn = a.D == 64 ? (const void*)k_attn<64> : a.D == 32 ? (const void*)k_attn<32> : nullptr;
    if (!fn) return hipErrorInvalidValue;
    if (lds > 64 * 1024) {
        const hipError_t e = hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
        if (e != hipSuccess) return e;
    }
    if (a.D == 64) hipLaunchKernelGGL(k_attn<64>, dim3(a.n_kv, M), dim3(256), lds, s, a);
    else hipLaunchKernelGGL(k_attn<32>, dim3(a.n_kv, M), dim3(256), lds, s, a);
    return hipGetLastError();
}

hipError_t launch_final(int M, const final_args& a, hipStream_t s) {
    const size_t lds = sizeof(float) * (size_t)a.E;
    if (M == 1) hipLaunchKernelGGL(k_final<1>, dim3(1), dim3(256), lds, s, a);
    else if (M == 2) hipLaunchKernelGGL(k_final<2>, dim3(1), dim3(256), lds, s, a);
    else return hipErrorInvalidValue;
    return hipGetLastError();
}

hipError_t launch_expf(const float* x, float* y, long long n, hipStream_t s) {
    hipLaunchKernelGGL(k_expf, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, x, y, n);
    return hipGetLastError();
}

}  // namespace sh
