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

// ---------------------------------------------------------------- Q4_0 GEMV
// One wave per block; a unit is UG groups of 8 rows (R rows).
// Phase 1, lanes over input blocks: lane j owns blocks j, j + 64, ... (< nb); it cuts them itself (int8 codes stay in
// registers) and, per row, loads its 16 B of codes (one row = 1 KB per load for the wave) and the 8 rows' scales of
// the block (16 B), and computes each (row, block) integer dot exactly. The dots and scales go to LDS.
// Phase 2, lanes over rows: lane (m, k) runs imi's per-row chain over blocks j in order
// (imi/core/tables.cpp:127-143): acc = fma(float(isum), d * dx, acc), cor = fma(d, s, cor), out = acc - 8 cor
// (q4x8, imi/kernels/q4x8.cpp:51-77: cor = fma(d, corr, cor), out = acc - cor) -- the same fp32 operations in the
// same order as the CPU, so the outputs are the CPU's bit for bit.
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
                    if (tok >= 0) q4_dequant_block(a.emb, tok, lane, xv);
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
            u32x4 c[8][NBL], s8[NBL];
#pragma unroll
            for (int b = 0; b < NBL; b++) {
                const int blk = lane + 64 * b;
                if (blk < nb) {
#pragma unroll
                    for (int r = 0; r < 8; r++) c[r][b] = __builtin_nontemporal_load(codes + (size_t)(8 * g + r) * nb + blk);
                    s8[b] = __builtin_nontemporal_load(scales + (size_t)g * nb + blk);
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
                cor = fmaf(d, sv[j], cor);
            }
            outv = PRO == PRO_CUT_HALF_AWAY ? acc - cor : fmaf(-8.0f, cor, acc);
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
                float* st = a.P->conv[m] + (size_t)a.conv_layer * dc * E;
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
template <int M, bool HALF, int NB>
__global__ __launch_bounds__(256) void k_gemv_cut(gemv_args a) {
    constexpr int TPB = 256 / NB, VPT = 32 / TPB, RPT = NB / 32, ST = NB + 4;
    extern __shared__ __align__(16) float lds[];
    int* l_xq = (int*)lds;                      // [M][NB][8] int8 codes of the cut input, 4 per word
    float* l_dx = lds + M * NB * 8;             // [M][NB]
    float* l_s = l_dx + M * NB;                 // [M][ST] s = d * sum (q4x8: 8 * d * sum)
    float* l_op = l_s + M * ST;                 // [M][8][ST] float(isum)
    float* l_oq = l_op + M * 8 * ST;            // [M][8][ST] d * dx
    float* l_dd = l_oq + M * 8 * ST;            // [8][ST] d
    const int t = threadIdx.x, lane = t & 63, g = blockIdx.x;
    // input share first: block jc, values part * VPT .. + VPT - 1
    const int jc = t / TPB, part = t - jc * TPB;
    f32x4 xin[M][VPT / 4];
#pragma unroll
    for (int m = 0; m < M; m++) {
        const f32x4* src = (const f32x4*)(a.src + (size_t)m * a.src_ld + 32 * jc + VPT * part);
#pragma unroll
        for (int k = 0; k < VPT / 4; k++) xin[m][k] = src[k];
    }
    // then the weights: rows sub * RPT .. + RPT - 1 of block jw
    const int jw = t % NB, sub = t / NB;
    u32x4 c[RPT];
    const u32x4* codes = (const u32x4*)a.W.codes + (size_t)(8 * g + sub * RPT) * NB + jw;
#pragma unroll
    for (int k = 0; k < RPT; k++) c[k] = __builtin_nontemporal_load(codes + (size_t)k * NB);
    const u32x4 s8 = __builtin_nontemporal_load((const u32x4*)a.W.scales + (size_t)g * NB + jw);
    // the cut of block jc by its TPB threads
#pragma unroll
    for (int m = 0; m < M; m++) {
        float v[VPT];
#pragma unroll
        for (int k = 0; k < VPT / 4; k++) {
            v[4 * k] = xin[m][k].x; v[4 * k + 1] = xin[m][k].y; v[4 * k + 2] = xin[m][k].z; v[4 * k + 3] = xin[m][k].w;
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
            l_dd[r * ST + jw] = d[k];
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
        for (int q0 = 0; q0 < NB / 4; q0 += 16) {   // per 64 blocks: the reads of the next 6 quads in flight
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
    }
    const float cor = __shfl(chain, (lane + 8 * M) & 63);
    if (acc_lane) {
        const int m = lane >> 3, r = lane & 7;
        a.out[(size_t)m * a.out_ld + 8 * g + r] = HALF ? chain - cor : fmaf(-8.0f, cor, chain);
    }
}

static size_t gemv_cut_lds(int M, int nb) {
    const size_t st = (size_t)nb + 4;
    return sizeof(float) * ((size_t)M * nb * 8 + (size_t)M * nb + (size_t)M * st + (size_t)2 * M * 8 * st + 8 * st);
}

// dynamic LDS bytes of a k_gemv instantiation
static size_t gemv_lds(int M, int UG, int nb, int E, bool norm) {
    const int R = 8 * UG;
    return sizeof(float) * ((size_t)nb * (M * R + 1) + (size_t)nb * (R + 1) + 2 * (size_t)M * nb + (norm ? (size_t)E : 0));
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
    uint16_t* kc = a.P->kc[m] + ((size_t)a.layer_ai * a.n_kv + g) * a.n_ctx * D;
    uint16_t* vc = a.P->vc[m] + ((size_t)a.layer_ai * a.n_kv + g) * a.n_ctx * D;
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
        const uint16_t* kt = kc + (size_t)(s0 + t) * D;
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
        int best = -1;
        if (a.part_v) {
            float v = -INFINITY;
            int bi = 0x7fffffff;
            for (int k = tid; k < a.n_part; k += 256) {
                const float ov = a.part_v[m * a.n_part + k];
                const int oi = a.part_i[m * a.n_part + k];
                if (ov > v || (ov == v && oi < bi)) { v = ov; bi = oi; }
            }
            red_v[tid] = v;
            red_i[tid] = bi;
            __syncthreads();
            for (int o = 128; o > 0; o >>= 1) {
                if (tid < o) {
                    const float ov = red_v[tid + o];
                    const int oi = red_i[tid + o];
                    if (ov > red_v[tid] || (ov == red_v[tid] && oi < red_i[tid])) { red_v[tid] = ov; red_i[tid] = oi; }
                }
                __syncthreads();
            }
            best = red_i[0];
            __syncthreads();
        }
        if (tid == 0) {
            a.P->best[m] = best;
            if (a.advance) {
                if (a.P->greedy && a.P->out_tok[m]) a.P->out_tok[m][a.P->n_done] = best;
                if (a.P->greedy) a.P->token[m] = best;
                a.P->pos[m] += 1;
            }
        }
    }
    if (tid == 0 && a.advance) a.P->n_done += 1;
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

hipError_t launch_gemv(int M, int pro, int epi, int grid, const gemv_args& a, hipStream_t s, hipEvent_t t0, hipEvent_t t1) {
    const int nbl = (a.W.nb + 63) / 64;
    const int ug = epi == EPI_SWIGLU ? 2 : epi == EPI_CONV ? 3 : 1;
    // the plain tables (input cut, rows stored): one workgroup per 8-row group, the grid is the group count
    const int nb = a.W.nb;
    if (epi == EPI_STORE && (pro == PRO_CUT || pro == PRO_CUT_HALF_AWAY) && (nb == 64 || nb == 128 || nb == 256) &&
        a.W.rows % 8 == 0 && (M == 1 || (M == 2 && pro == PRO_CUT))) {
        const bool half = pro == PRO_CUT_HALF_AWAY;
        const void* fn = nullptr;
#define SH_CUT_FN(M_, H_, NB_) if (M == M_ && half == H_ && nb == NB_) fn = (const void*)k_gemv_cut<M_, H_, NB_>;
        SH_CUT_FN(1, false, 64) SH_CUT_FN(1, false, 128) SH_CUT_FN(1, false, 256)
        SH_CUT_FN(1, true, 64) SH_CUT_FN(1, true, 128) SH_CUT_FN(1, true, 256)
        SH_CUT_FN(2, false, 64) SH_CUT_FN(2, false, 128) SH_CUT_FN(2, false, 256)
#undef SH_CUT_FN
        void* args[] = {const_cast<gemv_args*>(&a)};
        const dim3 gr(a.W.rows / 8), bl(256);
        const size_t lds = gemv_cut_lds(M, nb);
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

hipError_t launch_q4_rows(const q4dev& T, const int32_t* ids, int n, float* out, hipStream_t s) {
    hipLaunchKernelGGL(k_q4_rows, dim3(n), dim3(64), 0, s, T, ids, out);
    return hipGetLastError();
}

hipError_t launch_attn(int M, const attn_args& a, hipStream_t s) {
    const int grp = a.n_head / a.n_kv;
    const size_t lds = sizeof(float) * ((size_t)grp * a.D + (size_t)grp * a.n_ctx + 5 * (size_t)a.D + (size_t)grp);
    if (lds > 160 * 1024) return hipErrorInvalidValue;
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
