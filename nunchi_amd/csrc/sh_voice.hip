// Kernels of the Q8_0 voice generator (imi/core/voice.cpp:90-206) for gfx950.
//
// A pass is: code embeddings + the frame's base (one kernel), then per layer the qkvg table with the ln1 norm folded
// into its input staging, bidirectional attention over the P positions (one workgroup per query head), the o table
// adding into the residual stream, the gate|up table with the ln2 norm in front and SiLU(gate) * up behind, the down
// table adding into the residual stream; then the word scores of the needed codebooks with the output and head
// norms folded into their input staging. Every operation order is the CPU path's, so results agree bit for bit.
#include "sh_device.h"
#include "sh_voice.h"

namespace sh {
namespace {

constexpr int VX_NJ = 32;    // 32-column blocks per staged chunk of the input (1024 columns)
constexpr int VX_SS = 33;    // row stride of the per-block partial sums in LDS (odd: conflict-free column reads)

__host__ __device__ constexpr int vx_pp(int P) { return (P + 3) & ~3; }          // positions padded to float4
__host__ __device__ constexpr int vx_xj(int P) { return 32 * vx_pp(P) + 4; }     // floats per staged block

// rms scale of each position's input row (imi/core/vec.h:20-33), one wave per row
template <int P>
__device__ __forceinline__ void position_scales(const vtab_args& a, float* scl) {
    const int w = threadIdx.x >> 6, lane = threadIdx.x & 63;
    for (int p = w; p < P; p += VX_THREADS / 64) {
        const float* row = a.src + (size_t)p * a.src_ld;
        const float s = a.W.cols == 1024 ? rms_scale_wave_g<32>(row, a.eps) : rms_scale_wave(row, a.W.cols, a.eps);
        if (lane == 0) scl[p] = s;
    }
}

// columns [1024 q, 1024 q + 32 nbc) of the P positions, k-major: xs[block][column in block][position]
// (imi/core/voice.cpp:157-166: the transposed input, normed first when the table follows a norm)
// Thread t stages columns 4t..4t+3 of every position: all P 16-byte loads are in flight before the first LDS store
// (src rows and norm_w are 16-byte aligned, src_ld a multiple of 4: the launcher checks).
template <int P, int PRO>
__device__ __forceinline__ void stage_chunk(float* xs, const vtab_args& a, int q, int nbc, const float* scl) {
    constexpr int PP = vx_pp(P), XJ = vx_xj(P);
    static_assert(4 * VX_THREADS == 32 * VX_NJ, "one float4 of each position per thread");
    const int n = 32 * nbc, c0 = q * 32 * VX_NJ, k = 4 * threadIdx.x;
    if (k >= n) return;
    f32x4 v[P];
#pragma unroll
    for (int p = 0; p < P; p++) v[p] = *reinterpret_cast<const f32x4*>(a.src + (size_t)p * a.src_ld + c0 + k);
    f32x4 nw{};
    if (PRO == VP_NORM) nw = *reinterpret_cast<const f32x4*>(a.norm_w + c0 + k);
    float* dst = xs + (k >> 5) * XJ + (k & 31) * PP;
#pragma unroll
    for (int p = 0; p < P; p++) {
        float e[4] = {v[p].x, v[p].y, v[p].z, v[p].w};
        const float w4[4] = {nw.x, nw.y, nw.z, nw.w};
#pragma unroll
        for (int i = 0; i < 4; i++) {
            if (PRO == VP_NORM) e[i] = e[i] * scl[p] * w4[i];
            dst[i * PP + p] = e[i];
        }
    }
}

// results of the workgroup's NR rows (from group g0 on): thread t holds row t / P, position t % P
// et: this thread's entry of expf's table (thread t holds entry t % 32), requested when the kernel starts; the
// SwiGLU epilogue reads the table from LDS (no memory round trip at the end)
template <int P, int EPI, int NR>
__device__ __forceinline__ void table_epilogue(const vtab_args& a, int g0, float acc, float* ev, uint64_t et) {
    const int t = threadIdx.x, frow = t / P, fc = t - frow * P;
    if (EPI == VE_SWIGLU) {   // groups g0 (gate rows) and g0 + 1 (up rows): out[p][4 g0 + r] (voice.cpp:150-156)
        static_assert(EPI != VE_SWIGLU || NR == 16, "gate and up groups side by side");
        __shared__ uint64_t vE[32];
        if (t < 16 * P) ev[t] = acc;
        if (t < 32) vE[t] = et;
        __syncthreads();
        if (t < 8 * P) a.out[(size_t)fc * a.out_ld + 4 * g0 + frow] = silu_t(ev[t], vE) * ev[8 * P + t];
    } else {
        const int row = 8 * g0 + frow;
        if (t < NR * P && row < a.W.rows) {
            float* o = a.out + (size_t)fc * a.out_ld + row;
            *o = EPI == VE_RESID ? *o + acc : acc;   // x[i] += y[i] (voice.cpp:188,196)
        }
    }
}

// s[g][c] = sum over the block's 32 columns k of fma(w[g][k], x[k][c], s) in column order, for the R row groups'
// codes w (two 16-byte words each) and the staged block xb (column k, position c at xb[k * PP + c])
template <int P, int R>
__device__ __forceinline__ void block_sums(const float* xb, const u32x4 (&w)[R][2], float (&s)[R][P]) {
    constexpr int PP = vx_pp(P);
#pragma unroll
    for (int g = 0; g < R; g++)
#pragma unroll
        for (int c = 0; c < P; c++) s[g][c] = 0.0f;
#pragma unroll 4
    for (int kk = 0; kk < 32; kk++) {
        float xv[PP];
#pragma unroll
        for (int c4 = 0; c4 < PP / 4; c4++) {
            const f32x4 v = *reinterpret_cast<const f32x4*>(xb + kk * PP + 4 * c4);
            xv[4 * c4] = v.x; xv[4 * c4 + 1] = v.y; xv[4 * c4 + 2] = v.z; xv[4 * c4 + 3] = v.w;
        }
#pragma unroll
        for (int g = 0; g < R; g++) {
            const u32x4 h = w[g][kk >> 4];
            const unsigned word = (kk & 12) == 0 ? h.x : (kk & 12) == 4 ? h.y : (kk & 12) == 8 ? h.z : h.w;
            const float wf = (float)(int)(signed char)(word >> (8 * (kk & 3)));
#pragma unroll
            for (int c = 0; c < P; c++) s[g][c] = fmaf(wf, xv[c], s[g][c]);
        }
    }
}

// generic order (imi/core/tables.cpp:391-401): thread (row r of the group, block j) forms s = sum fma(w, x, s) over
// the block's 32 columns for every position; then thread (row, position) folds acc = fma(d, s, acc) block by block
template <int P, int PRO, int EPI>
__global__ __launch_bounds__(VX_THREADS) void k_vtab_gen(vtab_args a) {
    const uint64_t et = EPI == VE_SWIGLU ? kExp2Tab[threadIdx.x & 31] : 0;   // (first: its wait needs nothing later)
    constexpr int R = EPI == VE_SWIGLU ? 2 : 1;   // row groups per workgroup
    constexpr int PP = vx_pp(P), XJ = vx_xj(P);
    static_assert(8 * R * P <= VX_THREADS, "one folding thread per (row, position)");
    __shared__ __attribute__((aligned(16))) float xs[VX_NJ * XJ];
    __shared__ float ss[8 * R * P * VX_SS];
    __shared__ float ds[8 * R * VX_SS];
    __shared__ float scl[VX_MAX_P];
    __shared__ float ev[16 * VX_MAX_P];
    const int t = threadIdx.x, r8 = t & 7, jl = t >> 3;
    const int nb = a.W.nb, g0 = blockIdx.x * R;
    float acc = 0.0f;
    for (int q = 0; q * VX_NJ < nb; q++) {
        const int nbc = min(VX_NJ, nb - q * VX_NJ), j = q * VX_NJ + jl;
        u32x4 w[R][2];
        uint16_t dh[R];
        if (jl < nbc) {   // codes and scales first: their loads overlap the norm scales and the input staging
#pragma unroll
            for (int g = 0; g < R; g++) {
                const size_t blk = ((size_t)(g0 + g) * nb + j) * 8 + r8;
                const u32x4* cp = reinterpret_cast<const u32x4*>(a.W.codes + blk * 32);
                w[g][0] = cp[0];
                w[g][1] = cp[1];
                dh[g] = a.W.scales[blk];
            }
        }
        if (PRO == VP_NORM && q == 0) {
            position_scales<P>(a, scl);
            __syncthreads();
        }
        if (q) __syncthreads();   // the previous chunk's fold has read ss and ds
        stage_chunk<P, PRO>(xs, a, q, nbc, scl);
        if (jl < nbc) {
#pragma unroll
            for (int g = 0; g < R; g++) ds[(8 * g + r8) * VX_SS + jl] = h2f(dh[g]);
        }
        __syncthreads();
        if (jl < nbc) {
            float s[R][P];
            block_sums<P, R>(xs + jl * XJ, w, s);
#pragma unroll
            for (int g = 0; g < R; g++)
#pragma unroll
                for (int c = 0; c < P; c++) ss[((8 * g + r8) * P + c) * VX_SS + jl] = s[g][c];
        }
        __syncthreads();
        if (t < 8 * R * P) {
            const float* sp = ss + t * VX_SS;
            const float* dp = ds + (t / P) * VX_SS;
            for (int i = 0; i < nbc; i++) acc = fmaf(dp[i], sp[i], acc);
        }
    }
    table_epilogue<P, EPI, 8 * R>(a, g0, acc, ev, et);
}

// the generic order split over the input's 1024-column chunks, for tables wider than one chunk (the down table):
// workgroup (group g, chunk q) forms its blocks' sums s as k_vtab_gen does and stores them to
// part[g][8 P][nb] (row r8 * P + position c); k_vtab_fold then runs each (row, position)'s chain
// acc = fma(d, s, acc) over all blocks in order, so the results are k_vtab_gen's. Spreading the chunks over
// workgroups keeps the chip busy where one workgroup per group would walk the chunks one after another.
template <int P, int PRO>
__global__ __launch_bounds__(VX_THREADS) void k_vtab_part(vtab_args a) {
    constexpr int XJ = vx_xj(P);
    static_assert(8 * VX_NJ == VX_THREADS, "thread (row, block) of a chunk");
    __shared__ __attribute__((aligned(16))) float xs[VX_NJ * XJ];
    __shared__ float ss[8 * P * VX_SS];
    __shared__ float scl[VX_MAX_P];
    const int t = threadIdx.x, r8 = t & 7, jl = t >> 3;
    const int nb = a.W.nb, g = blockIdx.x, q = blockIdx.y;
    const int nbc = min(VX_NJ, nb - q * VX_NJ);
    u32x4 w[1][2];
    if (jl < nbc) {
        const size_t blk = ((size_t)g * nb + q * VX_NJ + jl) * 8 + r8;
        const u32x4* cp = reinterpret_cast<const u32x4*>(a.W.codes + blk * 32);
        w[0][0] = cp[0];
        w[0][1] = cp[1];
    }
    if (PRO == VP_NORM) {
        position_scales<P>(a, scl);
        __syncthreads();
    }
    stage_chunk<P, PRO>(xs, a, q, nbc, scl);
    __syncthreads();
    if (jl < nbc) {
        float s[1][P];
        block_sums<P, 1>(xs + jl * XJ, w, s);
#pragma unroll
        for (int c = 0; c < P; c++) ss[(r8 * P + c) * VX_SS + jl] = s[0][c];
    }
    __syncthreads();
    float* dst = a.part + (size_t)g * 8 * P * nb + q * VX_NJ;
    for (int i = t; i < 8 * P * VX_NJ; i += VX_THREADS) {
        const int row = i / VX_NJ, k = i - row * VX_NJ;
        if (k < nbc) dst[(size_t)row * nb + k] = ss[row * VX_SS + k];
    }
}

template <int P, int EPI>
__global__ __launch_bounds__(VX_THREADS) void k_vtab_fold(vtab_args a) {
    const uint64_t et = EPI == VE_SWIGLU ? kExp2Tab[threadIdx.x & 31] : 0;   // (first: its wait needs nothing later)
    __shared__ float ss[8 * P * VX_SS];
    __shared__ float ds[8 * VX_SS];
    __shared__ float ev[16 * VX_MAX_P];
    static_assert(VX_THREADS == 8 * VX_NJ, "thread (row, block) loads a chunk's scale");
    const int t = threadIdx.x, nb = a.W.nb, g0 = blockIdx.x, nq = (nb + VX_NJ - 1) / VX_NJ;
    const int k = t & (VX_NJ - 1), rw = t / VX_NJ;   // block k of rows rw, rw + 8, ... of the chunk; scale row rw
    const float* src = a.part + (size_t)g0 * 8 * P * nb;
    float v[P];
    uint16_t dh = 0;
    auto load = [&](int q) {   // chunk q into registers
        const bool in = q * VX_NJ + k < nb;
#pragma unroll
        for (int u = 0; u < P; u++) v[u] = in ? src[(size_t)(rw + 8 * u) * nb + q * VX_NJ + k] : 0.0f;
        if (in) dh = a.W.scales[((size_t)g0 * nb + q * VX_NJ + k) * 8 + rw];
    };
    load(0);
    float acc = 0.0f;
    for (int q = 0; q < nq; q++) {
        const int nbc = min(VX_NJ, nb - q * VX_NJ);
        if (q) __syncthreads();   // the previous chunk's fold has read ss and ds
#pragma unroll
        for (int u = 0; u < P; u++) ss[(rw + 8 * u) * VX_SS + k] = v[u];
        ds[rw * VX_SS + k] = h2f(dh);
        __syncthreads();
        if (q + 1 < nq) load(q + 1);
        if (t < 8 * P) {
            const float* sp = ss + t * VX_SS;
            const float* dp = ds + (t / P) * VX_SS;
            for (int i = 0; i < nbc; i++) acc = fmaf(dp[i], sp[i], acc);
        }
    }
    table_epilogue<P, EPI, 8>(a, g0, acc, ev, et);
}

// scaled order (imi/core/tables.cpp:324-365, P = 12 or 6): thread (row, position) runs one chain over all columns
// of fma(float(w) * d, x, acc); two row groups (16 rows) per workgroup. The workgroup stages 256 columns at a time,
// one chunk ahead: each thread loads one 16-byte word of codes (16 columns of one row's block) and the block's scale
// and stores the 16 products float(w) * d (exact: an int8 times an fp16 has at most 19 significant bits) to LDS, and
// the positions' inputs (normed first for a VP_NORM table) go position-major beside them; a chain step then reads
// 4 columns of its row and 4 of its position as one 16-byte LDS word each.
template <int P, int PRO, int EPI>
__global__ __launch_bounds__(VX_THREADS) void k_vtab_scaled(vtab_args a) {
    const uint64_t et = EPI == VE_SWIGLU ? kExp2Tab[threadIdx.x & 31] : 0;   // (first: its wait needs nothing later)
    constexpr int WC = 256, WS = WC + 4, NBK = WC / 32;   // columns per chunk, LDS row stride, blocks per chunk
    constexpr int NXQ = (P * (WC / 4) + VX_THREADS - 1) / VX_THREADS;   // input 16-byte words per thread per chunk
    static_assert(16 * P <= VX_THREADS && 2 * NBK * 8 * 2 == VX_THREADS, "one code word per thread per chunk");
    __shared__ __attribute__((aligned(16))) float sW[2][16 * WS];
    __shared__ __attribute__((aligned(16))) float sX[2][P * WS];
    __shared__ float scl[VX_MAX_P];
    __shared__ float ev[16 * VX_MAX_P];
    const int t = threadIdx.x, rl = t / P, c = t - rl * P;
    const int nb = a.W.nb, K = a.W.cols, ng = a.W.rows_pad / 8, nch = (K + WC - 1) / WC, g0 = blockIdx.x * 2;
    // staging role: group gg, block jb of the chunk, row r8 of the group, half h of the block's 32 codes
    const int gg = t >> 7, jb = (t >> 4) & 7, r8 = (t >> 1) & 7, h = t & 1;
    const int grp = min(g0 + gg, ng - 1);   // (a workgroup's second group past the table reads the last one; dropped)
    if (PRO == VP_NORM) {
        position_scales<P>(a, scl);
        __syncthreads();
    }
    u32x4 gq;
    uint16_t gs;
    f32x4 gx[NXQ];
    auto fetch = [&](int q) {   // every load unconditional, indices clamped into the buffers
        const int j = min(q * NBK + jb, nb - 1);
        const size_t blk = ((size_t)grp * nb + j) * 8 + r8;
        gq = reinterpret_cast<const u32x4*>(a.W.codes + blk * 32)[h];
        gs = a.W.scales[blk];
#pragma unroll
        for (int s = 0; s < NXQ; s++) {
            const int idx = min(t + VX_THREADS * s, P * (WC / 4) - 1), p = idx / (WC / 4), k = min(q * WC + 4 * (idx % (WC / 4)), K - 4);
            gx[s] = *reinterpret_cast<const f32x4*>(a.src + (size_t)p * a.src_ld + k);
        }
    };
    auto stash = [&](int b, int q) {
        const bool ok = q * NBK + jb < nb;   // a block past the table's columns stores zeros (never read)
        const float d = h2f(gs);
        const unsigned wv[4] = {gq.x, gq.y, gq.z, gq.w};
        float* dst = &sW[b][(8 * gg + r8) * WS + 32 * jb + 16 * h];
#pragma unroll
        for (int i = 0; i < 4; i++) {
            f32x4 o;
            o.x = ok ? (float)(int)(signed char)(wv[i] & 0xFFu) * d : 0.0f;
            o.y = ok ? (float)(int)(signed char)((wv[i] >> 8) & 0xFFu) * d : 0.0f;
            o.z = ok ? (float)(int)(signed char)((wv[i] >> 16) & 0xFFu) * d : 0.0f;
            o.w = ok ? (float)(int)(signed char)(wv[i] >> 24) * d : 0.0f;
            *reinterpret_cast<f32x4*>(dst + 4 * i) = o;
        }
#pragma unroll
        for (int s = 0; s < NXQ; s++) {
            const int idx = t + VX_THREADS * s;
            if (idx < P * (WC / 4)) {
                const int p = idx / (WC / 4), k4 = idx % (WC / 4), col = q * WC + 4 * k4;
                f32x4 e = gx[s];
                if (PRO == VP_NORM && col < K) {
                    const f32x4 nw = *reinterpret_cast<const f32x4*>(a.norm_w + col);
                    e.x = e.x * scl[p] * nw.x; e.y = e.y * scl[p] * nw.y;
                    e.z = e.z * scl[p] * nw.z; e.w = e.w * scl[p] * nw.w;
                }
                *reinterpret_cast<f32x4*>(&sX[b][p * WS + 4 * k4]) = e;
            }
        }
    };
    fetch(0);
    stash(0, 0);
    __syncthreads();
    float acc = 0.0f;
    const bool live = t < 16 * P;
    const int rr = live ? rl : 0, cc = live ? c : 0;
    for (int q = 0; q < nch; q++) {
        const int b = q & 1, nk4 = min(WC, K - q * WC) / 4;
        if (q + 1 < nch) fetch(q + 1);
        const float* wrow = &sW[b][rr * WS];
        const float* xrow = &sX[b][cc * WS];
        for (int k4 = 0; k4 < nk4; k4++) {
            const f32x4 w = *reinterpret_cast<const f32x4*>(wrow + 4 * k4);
            const f32x4 x = *reinterpret_cast<const f32x4*>(xrow + 4 * k4);
            acc = fmaf(w.x, x.x, acc);
            acc = fmaf(w.y, x.y, acc);
            acc = fmaf(w.z, x.z, acc);
            acc = fmaf(w.w, x.w, acc);
        }
        if (q + 1 < nch) stash(b ^ 1, q + 1);
        __syncthreads();
    }
    table_epilogue<P, EPI, 16>(a, g0, acc, ev, et);
}

// single-input order (imi/core/tables.cpp:366-382): 4 threads per row, thread o runs the chain over columns
// k % 4 == o of fma(float(w), d * x, a_o); the row's result is (a0 + a1) + (a2 + a3)
template <int HEAD>
__global__ __launch_bounds__(VX_THREADS) void k_vone(vone_args a, int cols) {
    __shared__ float xs[4096];
    const int nrb = (a.rows + 63) / 64, set = blockIdx.x / nrb, rb = blockIdx.x - set * nrb;
    int cb = 0;
    const float* src = a.src;
    if (HEAD) {   // the needed codebook's position: out_norm, then its head_norm (voice.cpp:199-203)
        if (set >= *a.n_need) return;
        cb = a.need[set];
        src = a.src + (size_t)cb * cols;
        const float s1 = cols == 1024 ? rms_scale_wave_g<32>(src, a.eps) : rms_scale_wave(src, cols, a.eps);
        for (int k = threadIdx.x; k < cols; k += VX_THREADS) xs[k] = src[k] * s1 * a.out_norm[k];
        __syncthreads();
        const float s2 = rms_scale_wave(static_cast<const float*>(xs), cols, a.eps);
        __syncthreads();
        const float* hn = a.head_norm + (size_t)cb * cols;
        for (int k = threadIdx.x; k < cols; k += VX_THREADS) xs[k] = xs[k] * s2 * hn[k];
    } else {
        for (int k = threadIdx.x; k < cols; k += VX_THREADS) xs[k] = src[k];
    }
    __syncthreads();
    const q8dev W = a.tabs[cb];
    const int o = threadIdx.x & 3, row = rb * 64 + (threadIdx.x >> 2);
    float acc = 0.0f;
    if (row < W.rows_pad) {
        const int g = row >> 3, r8 = row & 7, nb = W.nb;
        for (int j = 0; j < nb; j++) {
            const size_t blk = ((size_t)g * nb + j) * 8 + r8;
            const float d = h2f(W.scales[blk]);
            const u32x4* cp = reinterpret_cast<const u32x4*>(W.codes + blk * 32);
            const u32x4 h0 = cp[0], h1 = cp[1];
            const unsigned wd[8] = {h0.x, h0.y, h0.z, h0.w, h1.x, h1.y, h1.z, h1.w};
            const float* xb = xs + 32 * j + o;
#pragma unroll
            for (int q = 0; q < 8; q++) {
                const float wf = (float)(int)(signed char)(wd[q] >> (8 * o));
                acc = fmaf(wf, d * xb[4 * q], acc);
            }
        }
    }
    const float pair = acc + __shfl_xor(acc, 1);    // a0 + a1 (o = 0), a2 + a3 (o = 2)
    const float other = __shfl_xor(pair, 2);
    const float total = (o & 2) ? other + pair : pair + other;
    if (o == 0 && row < a.rows) a.out[(size_t)set * a.rows + row] = a.bias ? total + a.bias[row] : total;
}

// one query head per workgroup over the P positions (imi/core/voice.cpp:159-180): q/k rows rms-normed and rotated
// by position, scores fma-chained over the head width, softmax with a float sum, sigmoid head gate
__global__ __launch_bounds__(VX_THREADS) void k_vattn(vattn_args a) {
    __shared__ float qq[VX_MAX_P][VX_MAX_D], kk[VX_MAX_P][VX_MAX_D];
    __shared__ float sc[VX_MAX_P][VX_MAX_P + 1];
    __shared__ float sm[VX_MAX_P], gt[VX_MAX_P];
    __shared__ uint64_t vE[32];   // expf's table (an LDS copy: no memory round trip in the softmax)
    const int P = a.P, D = a.D, hh = blockIdx.x, kv = hh / (a.n_head / a.n_kv);
    const int Hq = a.n_head * D, Hk = a.n_kv * D, t = threadIdx.x;
    const uint64_t et = kExp2Tab[t & 31];   // (requested first, with the head gate's input)
    const float gin = a.qkv[(size_t)min(t, P - 1) * a.n_qkv + Hq + 2 * Hk + hh];
    for (int i = t; i < P * D; i += VX_THREADS) {
        const int p = i / D, e = i - p * D;
        const float* r = a.qkv + (size_t)p * a.n_qkv;
        qq[p][e] = r[hh * D + e];
        kk[p][e] = r[Hq + kv * D + e];
    }
    if (t < 32) vE[t] = et;
    __syncthreads();
    const int w = t >> 6, lane = t & 63, half = D / 2;
    for (int ri = w; ri < 2 * P; ri += VX_THREADS / 64) {
        const int p = ri < P ? ri : ri - P;
        float* v = ri < P ? kk[p] : qq[p];
        const float* nw = ri < P ? a.k_norm : a.q_norm;
        const float s = rms_scale_wave(static_cast<const float*>(v), D, a.eps);
        if (lane < half) {
            const float x0 = v[lane] * s * nw[lane], x1 = v[lane + half] * s * nw[lane + half];
            const float2 cs = a.rope_cs[p * half + lane];
            v[lane] = fmaf(x0, cs.x, -(x1 * cs.y));
            v[lane + half] = fmaf(x0, cs.y, x1 * cs.x);
        }
    }
    __syncthreads();
    if (t < P * P) {
        const int p = t / P, u = t - p * P;
        float s = 0.0f;
        for (int i = 0; i < D; i++) s = fmaf(qq[p][i], kk[u][i], s);
        sc[p][u] = s * a.scale;
    }
    __syncthreads();
    if (t < P) {
        float mx = -__builtin_inff();
        for (int u = 0; u < P; u++) mx = mx < sc[t][u] ? sc[t][u] : mx;   // std::max(mx, sc)
        float sum = 0.0f;
        for (int u = 0; u < P; u++) {
            const float e = expf_glibc_t(sc[t][u] - mx, vE);
            sc[t][u] = e;
            sum += e;
        }
        sm[t] = sum;
        gt[t] = 1.0f / (1.0f + expf_glibc_t(-gin, vE));
    }
    __syncthreads();
    for (int i = t; i < P * D; i += VX_THREADS) {
        const int p = i / D, e = i - p * D;
        const float* vcol = a.qkv + Hq + Hk + kv * D + e;
        float acc = 0.0f;
        for (int u = 0; u < P; u++) acc = fmaf(sc[p][u], vcol[(size_t)u * a.n_qkv], acc);
        a.att[(size_t)p * Hq + hh * D + e] = acc / sm[p] * gt[p];
    }
}

// pass input: position p's code row of codebook p (dequantized d * q), or mask_embd, plus the frame's base
// (imi/core/voice.cpp:122-127)
__global__ __launch_bounds__(VX_THREADS) void k_vembed(vembed_args a) {
    const int i = blockIdx.x * VX_THREADS + threadIdx.x;
    if (i >= a.P * a.E) return;
    const int p = i / a.E, e = i - p * a.E, code = a.codes[p];
    float v;
    if (code >= 0) {
        const q8dev T = a.tabs[p];
        const size_t blk = ((size_t)(code >> 3) * T.nb + (e >> 5)) * 8 + (code & 7);
        v = h2f(T.scales[blk]) * (float)T.codes[blk * 32 + (e & 31)];
    } else {
        v = a.mask[e];
    }
    a.x[i] = v + a.base[i];
}

// the brain's next input: the sum over codebooks, in order, of the chosen codes' feedback rows (voice.cpp:90-97)
__global__ __launch_bounds__(VX_THREADS) void k_vfeed(vfeed_args a) {
    const int i = blockIdx.x * VX_THREADS + threadIdx.x;
    if (i >= a.n_in) return;
    float o = 0.0f;
    for (int c = 0; c < a.n_cb; c++) {
        const uint8_t* blk = a.rows + (size_t)(a.codes[c] + c * a.n_vocab) * a.row_bytes + (size_t)(i >> 5) * 34;
        const float d = h2f(*reinterpret_cast<const uint16_t*>(blk));
        const float v = d * (float)(signed char)blk[2 + (i & 31)];
        o = o + v;
    }
    a.out[i] = o;
}

// One workgroup per scored codebook j (imi_talker::next, imi/core/talk.cpp:147-164). The row is read into LDS; the
// repeat penalty goes once to each distinct code of the history window: every frame offers its index to first[c]
// (an LDS minimum), and the frame that holds the minimum applies the penalty. The maximum is reduced across the
// workgroup (exact in any order), p[v] = exp((double)(l[v] - max) / temp) is formed in parallel, and thread 0 then
// runs imi's two in-order loops in double: the sum, and r = u * sum minus p[0], p[1], ... until r <= 0, which names
// the pick. Thread 0 takes p 16 values at a time: the LDS reads overlap, and the pick loop tests a block at once.
__global__ __launch_bounds__(256) void k_vsample(vsample_args a) {
    constexpr int VB = 16;
    extern __shared__ __attribute__((aligned(16))) unsigned char vs_lds[];
    double* ps = reinterpret_cast<double*>(vs_lds);                 // [V]
    int* first = reinterpret_cast<int*>(vs_lds);                    // [V], in ps's room until p is formed
    float* lf = reinterpret_cast<float*>(ps + a.V);                 // [V]
    int* hc = reinterpret_cast<int*>(lf + a.V);                     // [VS_MAX_HIST]
    __shared__ float wmax[4];
    const int j = blockIdx.x, t = threadIdx.x, V = a.V;
    if (j >= *a.n_need) return;
    const int cb = a.need[j];
    float* l = a.scores + (size_t)j * V;
    for (int v = t; v < V; v += 256) {
        lf[v] = l[v];
        first[v] = VS_MAX_HIST;
    }
    for (int f = t; f < a.n_frames; f += 256) hc[f] = a.hist[(size_t)f * a.n_cb + cb];
    __syncthreads();
    for (int f = t; f < a.n_frames; f += 256) {
        const int c = hc[f];
        if (c >= 0 && c < V) atomicMin(&first[c], f);
    }
    __syncthreads();
    for (int f = t; f < a.n_frames; f += 256) {
        const int c = hc[f];
        if (c >= 0 && c < V && first[c] == f) lf[c] = lf[c] > 0 ? lf[c] / a.rep : lf[c] * a.rep;
    }
    __syncthreads();
    float m = -INFINITY;
    for (int v = t; v < V; v += 256) m = fmaxf(m, lf[v]);
    m = wave_max(m);
    if ((t & 63) == 0) wmax[t >> 6] = m;
    __syncthreads();
    const float lmax = fmaxf(fmaxf(wmax[0], wmax[1]), fmaxf(wmax[2], wmax[3]));
    const double temp = a.temp;
    for (int v = t; v < V; v += 256) {
        ps[v] = exp((double)(lf[v] - lmax) / temp);
        l[v] = lf[v];
    }
    __syncthreads();
    if (t == 0) {
        const int VF = V & ~(VB - 1);   // whole blocks of VB codes; the rest one by one
        double sum = 0;
        for (int v0 = 0; v0 < VF; v0 += VB) {
            double b[VB];
#pragma unroll
            for (int i = 0; i < VB; i++) b[i] = ps[v0 + i];
#pragma unroll
            for (int i = 0; i < VB; i++) sum += b[i];
        }
        for (int v = VF; v < V; v++) sum += ps[v];
        double r = a.u[j] * sum;
        int pick = -1;
        // per block: the VB subtractions in order (no branch), then the first partial r <= 0 among them; the
        // subtractions past that one change nothing, as imi stops there
        for (int v0 = 0; v0 < VF && pick < 0; v0 += VB) {
            double b[VB], rr[VB];
#pragma unroll
            for (int i = 0; i < VB; i++) b[i] = ps[v0 + i];
#pragma unroll
            for (int i = 0; i < VB; i++) {
                r -= b[i];
                rr[i] = r;
            }
            int hit = VB;
#pragma unroll
            for (int i = VB - 1; i >= 0; i--) hit = rr[i] <= 0 ? i : hit;
            if (hit < VB) pick = v0 + hit;
        }
        for (int v = VF; v < V && pick < 0; v++) {
            r -= ps[v];
            if (r <= 0) pick = v;
        }
        if (pick < 0) pick = V - 1;
        a.picks[j] = pick;
        a.keep[j] = 1.0 - ps[V - 1] / sum;
    }
}

template <int P, int PRO, int EPI>
hipError_t launch_vtab_p(const vtab_args& a, hipStream_t s) {
    if constexpr (P == 6 || P == 12)
        hipLaunchKernelGGL((k_vtab_scaled<P, PRO, EPI>), dim3(a.units), dim3(VX_THREADS), 0, s, a);
    else {
        if constexpr (EPI != VE_SWIGLU) {
            if (a.part && a.W.nb > VX_NJ) {
                hipLaunchKernelGGL((k_vtab_part<P, PRO>), dim3(a.units, (a.W.nb + VX_NJ - 1) / VX_NJ),
                                   dim3(VX_THREADS), 0, s, a);
                hipLaunchKernelGGL((k_vtab_fold<P, EPI>), dim3(a.units), dim3(VX_THREADS), 0, s, a);
                return hipGetLastError();
            }
        }
        hipLaunchKernelGGL((k_vtab_gen<P, PRO, EPI>), dim3(a.units), dim3(VX_THREADS), 0, s, a);
    }
    return hipGetLastError();
}

template <int P>
hipError_t launch_vtab_kind(int pro, int epi, const vtab_args& a, hipStream_t s) {
    if (pro == VP_NORM && epi == VE_STORE) return launch_vtab_p<P, VP_NORM, VE_STORE>(a, s);
    if (pro == VP_PLAIN && epi == VE_RESID) return launch_vtab_p<P, VP_PLAIN, VE_RESID>(a, s);
    if (pro == VP_NORM && epi == VE_SWIGLU) return launch_vtab_p<P, VP_NORM, VE_SWIGLU>(a, s);
    if (pro == VP_PLAIN && epi == VE_STORE) return launch_vtab_p<P, VP_PLAIN, VE_STORE>(a, s);
    return hipErrorInvalidValue;
}

}  // namespace

hipError_t launch_vsample(const vsample_args& a, int max_need, hipStream_t s) {
    if (a.V < 1 || a.V > VS_MAX_V || a.n_frames < 0 || a.n_frames > VS_MAX_HIST || max_need < 1) return hipErrorInvalidValue;
    const size_t lds = (size_t)a.V * 8 + (size_t)a.V * 4 + VS_MAX_HIST * 4;
    hipLaunchKernelGGL(k_vsample, dim3(max_need), dim3(256), lds, s, a);
    return hipGetLastError();
}

hipError_t launch_vtab(int P, int pro, int epi, const vtab_args& a, hipStream_t s) {
    // the input staging reads 16-byte words of every position's row and of the norm weights
    if (a.src_ld % 4 || reinterpret_cast<uintptr_t>(a.src) % 16 ||
        (pro == VP_NORM && reinterpret_cast<uintptr_t>(a.norm_w) % 16))
        return hipErrorInvalidValue;
    switch (P) {
        case 2: return launch_vtab_kind<2>(pro, epi, a, s);
        case 3: return launch_vtab_kind<3>(pro, epi, a, s);
        case 4: return launch_vtab_kind<4>(pro, epi, a, s);
        case 5: return launch_vtab_kind<5>(pro, epi, a, s);
        case 6: return launch_vtab_kind<6>(pro, epi, a, s);
        case 7: return launch_vtab_kind<7>(pro, epi, a, s);
        case 8: return launch_vtab_kind<8>(pro, epi, a, s);
        case 9: return launch_vtab_kind<9>(pro, epi, a, s);
        case 10: return launch_vtab_kind<10>(pro, epi, a, s);
        case 11: return launch_vtab_kind<11>(pro, epi, a, s);
        case 12: return launch_vtab_kind<12>(pro, epi, a, s);
        default: return hipErrorInvalidValue;
    }
}

hipError_t launch_vone(const vone_args& a, int n_sets, int cols, hipStream_t s) {
    if (cols > 4096 || cols % 32) return hipErrorInvalidValue;
    const int grid = n_sets * ((a.rows + 63) / 64);
    if (a.head)
        hipLaunchKernelGGL(k_vone<1>, dim3(grid), dim3(VX_THREADS), 0, s, a, cols);
    else
        hipLaunchKernelGGL(k_vone<0>, dim3(grid), dim3(VX_THREADS), 0, s, a, cols);
    return hipGetLastError();
}

hipError_t launch_vattn(const vattn_args& a, hipStream_t s) {
    if (a.P > VX_MAX_P || a.D > VX_MAX_D || a.D % 32) return hipErrorInvalidValue;
    hipLaunchKernelGGL(k_vattn, dim3(a.n_head), dim3(VX_THREADS), 0, s, a);
    return hipGetLastError();
}

hipError_t launch_vembed(const vembed_args& a, hipStream_t s) {
    hipLaunchKernelGGL(k_vembed, dim3((a.P * a.E + VX_THREADS - 1) / VX_THREADS), dim3(VX_THREADS), 0, s, a);
    return hipGetLastError();
}

hipError_t launch_vfeed(const vfeed_args& a, hipStream_t s) {
    hipLaunchKernelGGL(k_vfeed, dim3((a.n_in + VX_THREADS - 1) / VX_THREADS), dim3(VX_THREADS), 0, s, a);
    return hipGetLastError();
}

}  // namespace sh
