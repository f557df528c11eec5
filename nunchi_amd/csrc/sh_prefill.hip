// Prefill kernels (imi_seoul::step_batch / run_batch, imi/core/seoul.cpp:490-655) for gfx950.
//
// Per layer: the table products run on the int8 matrix cores, everything between them (norms, cuts, the short conv,
// attention) as per-position kernels. Every fp32 operation is the one imi's CPU path does for that position, in the
// same order, so hidden states and word scores equal n single steps bit for bit.
#include "sh_device.h"
#include "sh_prefill.h"

#include <algorithm>
#include <cstdlib>

namespace sh {
namespace {

typedef int i32x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ void load32(const float* p, float* v) {
    const f32x4* q = reinterpret_cast<const f32x4*>(p);
#pragma unroll
    for (int k = 0; k < 8; k++) { const f32x4 t = q[k]; v[4 * k] = t.x; v[4 * k + 1] = t.y; v[4 * k + 2] = t.z; v[4 * k + 3] = t.w; }
}

// cut 32 floats (imi/core/vec.h:47-75, round half to even) into block j of position p of a block-major cut
__device__ __forceinline__ void cut_store(const pf_cut& c, int n, int j, int p, const float* v) {
    int q8[8], sum;
    const float d = cut32(v, q8, &sum, false);
    u32x4* qp = reinterpret_cast<u32x4*>(c.q + ((size_t)j * n + p) * 32);
    qp[0] = u32x4{(unsigned)q8[0], (unsigned)q8[1], (unsigned)q8[2], (unsigned)q8[3]};
    qp[1] = u32x4{(unsigned)q8[4], (unsigned)q8[5], (unsigned)q8[6], (unsigned)q8[7]};
    c.d[(size_t)j * n + p] = d;
    c.s[(size_t)j * n + p] = d * (float)sum;
}

// the conv memory after a batch (imi/core/seoul.cpp:562-577): tap tt of channel e becomes b x of position n - d_conv + tt,
// or, for a batch shorter than the memory, the memory's own tap tt + n; increasing tt reads only taps not yet rewritten
__device__ __forceinline__ void conv_state_update(const pf_conv_args& a, int e) {
    if (e >= a.E) return;
    const int ub = 24 * (e >> 3) + (e & 7), dc = a.d_conv, E = a.E;
    for (int tt = 0; tt < dc; tt++) {
        const int q = a.n - dc + tt;
        float v;
        if (q >= 0) {
            const float* rq = a.bcx + (size_t)q * 3 * E + ub;
            v = rq[0] * rq[16];
        } else {
            v = a.state[(size_t)(tt + a.n) * E + e];
        }
        a.state[(size_t)tt * E + e] = v;
    }
}

// ---------------------------------------------------------------- per-position norms
// PFR_FIRST: x = the word's dequantized row (Q4_0: (code - 8) * d; Q6_K: imi_q6k_dequant_row) or the given embedding
// row (imi/core/seoul.cpp:363-364);
// PFR_RESID: x = fma(y * rms(y), w_post, x) (imi/core/vec.h:41-44); then h = x * rms(x) * w_pre, cut or stored
// One wave per position, PFR_PPW positions per workgroup (no workgroup barriers): the wave stages its rows in LDS,
// runs both norms' chains (rms_scale_wave, imi's AVX2 order) and cuts its blocks, a block per lane. One position per
// workgroup spreads a window's positions over every compute unit: each position reads 32 KB (y, x and both norm
// weights), and 4 per workgroup on 112 units waited on the units' read rate (8.0 against 8.4 us per launch).
constexpr int PFR_PPW = 1;
template <int MODE>
__global__ __launch_bounds__(64 * PFR_PPW) void k_pf_rows(pf_rows_args a) {
    __shared__ __attribute__((aligned(16))) float xs_all[PFR_PPW][2048];
    __shared__ __attribute__((aligned(16))) float hs_all[PFR_PPW][2048];
    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6, p = blockIdx.x * PFR_PPW + wv, E = a.E, nb = E / 32;
    const int nwg = (a.n + PFR_PPW - 1) / PFR_PPW;
    if (MODE == PFR_RESID && (int)blockIdx.x >= nwg) {   // the conv memory update's workgroups (a.conv.state set)
        conv_state_update(a.conv, ((int)blockIdx.x - nwg) * 64 * PFR_PPW + (int)threadIdx.x);
        return;
    }
    if (p >= a.n) return;
    float* xs = xs_all[wv];
    float* hs = hs_all[wv];
    float* xr = a.x + (size_t)p * E;
    // the second norm's weights requested first too: behind the first norm they were one more memory round trip.
    // Every operand load is issued on every path (words past E re-read the last one, unused), so the compiler's
    // waits count exactly and never include the stores of x below
    constexpr int NQ2 = 2048 / 256;   // float4 words per lane at most
    float4 wq[NQ2];
#pragma unroll
    for (int q = 0; q < NQ2; q++) wq[q] = *reinterpret_cast<const float4*>(a.w_pre + min(4 * lane + 256 * q, E - 4));
    if (MODE == PFR_FIRST) {
        const int tok = a.tokens ? a.tokens[p] : -1;
        if (tok >= 0 && a.vocab6.codes) {
            for (int j = lane; j < nb; j += 64) q6k_dequant32((const u32x4*)a.vocab6.codes, a.vocab6.d, a.vocab6.nbk, tok, j, xs + 32 * j);
        } else if (tok >= 0) {
            for (int j = lane; j < nb; j += 64) {
                const u32x4 c = reinterpret_cast<const u32x4*>(a.vocab.codes)[(size_t)tok * nb + j];
                const float d = h2f(reinterpret_cast<const uint16_t*>(a.vocab.scales)[((size_t)(tok >> 3) * nb + j) * 8 + (tok & 7)]);
                const unsigned w[4] = {c.x, c.y, c.z, c.w};
#pragma unroll
                for (int i = 0; i < 16; i++) {
                    const unsigned byte = (w[i >> 2] >> (8 * (i & 3))) & 0xFFu;
                    xs[32 * j + i] = (float)((int)(byte & 15u) - 8) * d;
                    xs[32 * j + 16 + i] = (float)((int)(byte >> 4) - 8) * d;
                }
            }
        } else {
            for (int i = 4 * lane; i < E; i += 256)
                *reinterpret_cast<float4*>(xs + i) = *reinterpret_cast<const float4*>(a.embd + (size_t)p * E + i);
        }
        __builtin_amdgcn_wave_barrier();
        for (int i = 4 * lane; i < E; i += 256) *reinterpret_cast<float4*>(xr + i) = *reinterpret_cast<const float4*>(xs + i);
    } else {
        // every global operand of the position is requested first (one memory latency, not three)
        constexpr int NQ = 2048 / 256;   // float4 words per lane at most
        const float* yr = a.y + (size_t)p * E;
        float4 y4[NQ], x4[NQ], wp[NQ];
#pragma unroll
        for (int q = 0; q < NQ; q++) {
            const int i = min(4 * lane + 256 * q, E - 4);
            y4[q] = *reinterpret_cast<const float4*>(yr + i);
            x4[q] = *reinterpret_cast<const float4*>(xr + i);
            wp[q] = *reinterpret_cast<const float4*>(a.w_post + i);
        }
#pragma unroll
        for (int q = 0; q < NQ; q++)
            if (4 * lane + 256 * q < E) *reinterpret_cast<float4*>(hs + 4 * lane + 256 * q) = y4[q];
        __builtin_amdgcn_wave_barrier();
        const float sc1 = rms_scale_wave(static_cast<const float*>(hs), E, a.eps);
#pragma unroll
        for (int q = 0; q < NQ; q++) {
            const int i = 4 * lane + 256 * q;
            x4[q] = make_float4(fmaf(y4[q].x * sc1, wp[q].x, x4[q].x), fmaf(y4[q].y * sc1, wp[q].y, x4[q].y),
                                fmaf(y4[q].z * sc1, wp[q].z, x4[q].z), fmaf(y4[q].w * sc1, wp[q].w, x4[q].w));
            if (i < E) *reinterpret_cast<float4*>(xs + i) = x4[q];
        }
#pragma unroll
        for (int q = 0; q < NQ; q++) {   // (x to memory once every operand load has been consumed)
            const int i = 4 * lane + 256 * q;
            if (i < E) *reinterpret_cast<float4*>(xr + i) = x4[q];
        }
        __builtin_amdgcn_wave_barrier();
    }
    const float sc2 = rms_scale_wave(static_cast<const float*>(xs), E, a.eps);
#pragma unroll
    for (int q = 0; q < NQ2; q++) {
        const int i = 4 * lane + 256 * q;
        if (i < E) {
            const float4 x4 = *reinterpret_cast<const float4*>(xs + i), w4 = wq[q];
            const float4 h = make_float4(x4.x * sc2 * w4.x, x4.y * sc2 * w4.y, x4.z * sc2 * w4.z, x4.w * sc2 * w4.w);
            *reinterpret_cast<float4*>(hs + i) = h;
            if (a.hidden) *reinterpret_cast<float4*>(a.hidden + (size_t)p * E + i) = h;
        }
    }
    if (!a.cut.q) return;
    __builtin_amdgcn_wave_barrier();
    for (int j = lane; j < nb; j += 64) cut_store(a.cut, a.n, j, p, hs + 32 * j);
}

// ---------------------------------------------------------------- cut of n rows
__global__ __launch_bounds__(256) void k_pf_cut(pf_cutk_args a) {
    const int nb = a.K / 32, idx = blockIdx.x * 256 + threadIdx.x;
    if (idx >= a.n * nb) return;
    const int j = idx / a.n, p = idx - j * a.n;
    float v[32];
    load32(a.src + (size_t)p * a.ld + 32 * j, v);
    cut_store(a.cut, a.n, j, p, v);
}

// ---------------------------------------------------------------- table products on the matrix cores
// Workgroup tile 64 rows x 64 positions, wave tile 32 x 32 (2 x 2 products of 16 x 16 per 32-column block).
// v_mfma_i32_16x16x32_i8 operands: lane l holds row / position l % 16, columns 8 (l / 16) .. + 7 of the block;
// the result's lane l holds rows 4 (l / 16) + i (i < 4) at position l % 16. The weight codes enter as they are
// stored (0..15), the input as its int8 cut, so each product is imi's integer block sum exactly; then per (row,
// position), block by block in order: acc = fma(float(isum), d * dx, acc), cor = fma(d, s, cor), and at the end
// out = fma(-8, cor, acc) (imi/core/tables.cpp:419-454, the batch kernel imi's prefill uses); Q4_1 tables take the
// block minimum m in the cor chain and end as acc + cor.
template <int EPI, bool HM>
__global__ __launch_bounds__(256) void k_pf_gemm(pf_gemm_args a) {
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    const int li = lane & 15, lq = lane >> 4;
    const int rows = a.W.rows, n = a.n, nb = a.W.nb;
    const int rbase = blockIdx.x * 64 + (w & 1) * 32, pbase = blockIdx.y * 64 + (w >> 1) * 32;
    if (rbase >= rows || pbase >= n) return;   // whole waves; no barriers below
    const uint8_t* codes = static_cast<const uint8_t*>(a.W.codes);
    const uint16_t* scales = static_cast<const uint16_t*>(a.W.scales);
    const uint16_t* mins = static_cast<const uint16_t*>(a.W.mins);
    const uint8_t* ap[2];
    const uint16_t* dp[2];
    const uint16_t* mp[2];
#pragma unroll
    for (int mt = 0; mt < 2; mt++) {
        const int r = min(rbase + 16 * mt + li, rows - 1);              // operand row (clamped: results dropped)
        ap[mt] = codes + (size_t)r * nb * 16 + (lq & 1) * 8;            // bytes 0-7 or 8-15 of the row's block
        const int rd = min(rbase + 16 * mt + 4 * lq, rows - 4);         // first of the 4 result rows
        dp[mt] = scales + (size_t)(rd >> 3) * nb * 8 + (rd & 7);
        mp[mt] = HM ? mins + (size_t)(rd >> 3) * nb * 8 + (rd & 7) : dp[mt];
    }
    const int shift = (lq >> 1) * 4;   // columns 0-15: low nibbles, 16-31: high nibbles
    int pp[2];
#pragma unroll
    for (int nt = 0; nt < 2; nt++) pp[nt] = min(pbase + 16 * nt + li, n - 1);

    float acc[2][2][4], cor[2][2][4];
#pragma unroll
    for (int mt = 0; mt < 2; mt++)
#pragma unroll
        for (int nt = 0; nt < 2; nt++)
#pragma unroll
            for (int i = 0; i < 4; i++) { acc[mt][nt][i] = 0.0f; cor[mt][nt][i] = 0.0f; }

    // operands of block j, fetched one block ahead
    uint2 ra[2], rs[2], rm[2];
    long rb[2];
    float fx[2], fs[2];
    auto fetch = [&](int j) {
#pragma unroll
        for (int mt = 0; mt < 2; mt++) {
            ra[mt] = *reinterpret_cast<const uint2*>(ap[mt] + (size_t)j * 16);
            rs[mt] = *reinterpret_cast<const uint2*>(dp[mt] + (size_t)j * 8);
            if (HM) rm[mt] = *reinterpret_cast<const uint2*>(mp[mt] + (size_t)j * 8);
        }
#pragma unroll
        for (int nt = 0; nt < 2; nt++) {
            const size_t o = (size_t)j * n + pp[nt];
            rb[nt] = *reinterpret_cast<const long*>(a.in.q + o * 32 + lq * 8);
            fx[nt] = a.in.d[o];
            fs[nt] = a.in.s[o];
        }
    };
    fetch(0);
    for (int j = 0; j < nb; j++) {
        const uint2 ca[2] = {ra[0], ra[1]}, cs[2] = {rs[0], rs[1]}, cm[2] = {HM ? rm[0] : rs[0], HM ? rm[1] : rs[1]};
        const long cb[2] = {rb[0], rb[1]};
        const float cx[2] = {fx[0], fx[1]}, cz[2] = {fs[0], fs[1]};
        if (j + 1 < nb) fetch(j + 1);
        i32x4 isum[2][2];
#pragma unroll
        for (int mt = 0; mt < 2; mt++) {
            const unsigned lo = (ca[mt].x >> shift) & 0x0F0F0F0Fu, hi = (ca[mt].y >> shift) & 0x0F0F0F0Fu;
            const long av = (long)((unsigned long)lo | ((unsigned long)hi << 32));
#pragma unroll
            for (int nt = 0; nt < 2; nt++)
                isum[mt][nt] = __builtin_amdgcn_mfma_i32_16x16x32_i8(av, cb[nt], i32x4{0, 0, 0, 0}, 0, 0, 0);
        }
#pragma unroll
        for (int mt = 0; mt < 2; mt++) {
            const float dd[4] = {h2f((uint16_t)(cs[mt].x & 0xFFFFu)), h2f((uint16_t)(cs[mt].x >> 16)),
                                 h2f((uint16_t)(cs[mt].y & 0xFFFFu)), h2f((uint16_t)(cs[mt].y >> 16))};
            const float mm[4] = {h2f((uint16_t)(cm[mt].x & 0xFFFFu)), h2f((uint16_t)(cm[mt].x >> 16)),
                                 h2f((uint16_t)(cm[mt].y & 0xFFFFu)), h2f((uint16_t)(cm[mt].y >> 16))};
#pragma unroll
            for (int nt = 0; nt < 2; nt++)
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    acc[mt][nt][i] = fmaf((float)isum[mt][nt][i], dd[i] * cx[nt], acc[mt][nt][i]);
                    cor[mt][nt][i] = fmaf(mm[i], cz[nt], cor[mt][nt][i]);
                }
        }
    }
#pragma unroll
    for (int mt = 0; mt < 2; mt++)
#pragma unroll
        for (int nt = 0; nt < 2; nt++) {
            const int p = pbase + 16 * nt + li, r0 = rbase + 16 * mt + 4 * lq;
            float v[4];
#pragma unroll
            for (int i = 0; i < 4; i++) v[i] = HM ? acc[mt][nt][i] + cor[mt][nt][i] : fmaf(-8.0f, cor[mt][nt][i], acc[mt][nt][i]);
            if (EPI == EPI_SWIGLU) {
                // rows 0-7 of the 16-row tile are a gate group, rows 8-15 the matching up group (lanes + 32)
                float up[4];
#pragma unroll
                for (int i = 0; i < 4; i++) up[i] = __shfl_xor(v[i], 32);
                if (lq < 2 && p < n) {
                    float* o = a.out + (size_t)p * a.out_ld + (rbase + 16 * mt) / 2 + 4 * lq;
#pragma unroll
                    for (int i = 0; i < 4; i++) o[i] = silu(v[i]) * up[i];
                }
            } else if (p < n) {
                float* o = a.out + (size_t)p * a.out_ld + r0;
#pragma unroll
                for (int i = 0; i < 4; i++)
                    if (r0 + i < rows) o[i] = v[i];
            }
        }
}

// LDS-staged form of the same product (taken when nb is a multiple of KC): per workgroup the operands of KC blocks
// (64 rows of codes, their scales and, for Q4_1, minima; 64 positions of input codes and their (d, s)) are fetched
// with wide coalesced loads into registers while the waves run the previous KC blocks from LDS, then stored to the
// other half of a double buffer, the codes already split into their low and high nibbles. The per-(row, position)
// operations and their order are k_pf_gemm's; two of the three fp32 operations per (row, position, block) run on
// the matrix cores as K = 1 outer products, v_mfma_f32_16x16x1_4b_f32, whose four 16 x 16 blocks are the wave's
// (row tile, position tile) pairs: dd = d x dx (accumulator 0) and cor = fma(d, s, cor) (the running cor as the
// accumulator, one product per block in block order). That operation rounds once, like fmaf: it equals the VALU's
// fmaf bit for bit, denormals and the fused cancellation included (measured on 4.2 M cases); d x dx + 0 differs from
// the product only in the sign of a zero, which the acc chain (started at +0) cannot see. Only acc =
// fma(float(isum), dd, acc) stays on the VALU. A workgroup is 4 waves over 64 rows x 2 PW positions, a wave 32 rows x
// PW positions: PW = 32 for tables with enough rows, 16 for the narrow ones (2048 rows: two waves per SIMD instead of
// one), whose matrix-core blocks for the missing position tile are computed on a repeated position and dropped.
template <int EPI, bool HM, int KC, int PW>
__global__ __launch_bounds__(256, (KC == 4 && PW == 32) ? 3 : 2) void k_pf_gemm_lds(pf_gemm_args a) {
    typedef float v16f __attribute__((ext_vector_type(16)));
    constexpr int P = 2 * PW, NTW = PW / 16;          // positions per workgroup; 16-position tiles per wave
    constexpr int SA = 8 * KC + 2;                    // dwords per row: 32 nibble bytes per block + 2 (bank spread)
    __shared__ __align__(16) unsigned sA[2][64 * SA]; // row r, block j: low nibbles of its 16 code bytes, then high
    __shared__ u32x4 sB[2][KC][P][2];       // position p's 32 input codes of block j, 16-byte halves swapped when p & 8
    __shared__ __align__(16) uint16_t sD[2][KC][64];
    __shared__ __align__(16) uint16_t sM[2][KC][HM ? 64 : 8];
    __shared__ float2 sX[2][KC][P];         // (d, s) of position p's block j
    __shared__ uint64_t sE[EPI == EPI_SWIGLU ? 32 : 1];   // expf's table for the SwiGLU epilogue (an LDS copy)
    const int t = threadIdx.x, lane = t & 63, w = t >> 6, li = lane & 15, lq = lane >> 4;
    const int rows = a.W.rows, n = a.n, nb = a.W.nb, nch = nb / KC, ng = rows / 8;
    const int r0 = blockIdx.x * 64, p0 = blockIdx.y * P, rl = (w & 1) * 32, pl = (w >> 1) * PW;
    // staging words per thread (the (d, s) pairs of a narrow tile need only the first P * KC threads)
    constexpr int NA = 64 * KC / 256, NBQ = P * KC * 2 / 256, NX = (P * KC + 255) / 256;
    static_assert(NA >= 1 && NBQ >= 1 && 64 * KC % 256 == 0 && P * KC * 2 % 256 == 0, "KC too small for the staging");
    // this thread's staging sources, chunk 0 (rows and positions past the table / batch are clamped: their results
    // are dropped); chunk c adds c * KC blocks
    const u32x4* pa[NA];
    const u32x4* pb[NBQ];
    const float* px[NX];
#pragma unroll
    for (int q = 0; q < NA; q++) {
        const int idx = t + 256 * q;
        pa[q] = (const u32x4*)a.W.codes + (size_t)min(r0 + idx / KC, rows - 1) * nb + idx % KC;
    }
#pragma unroll
    for (int q = 0; q < NBQ; q++) {
        const int idx = t + 256 * q, rem = idx % (2 * P);
        pb[q] = (const u32x4*)a.in.q + ((size_t)(idx / (2 * P)) * n + min(p0 + (rem >> 1), n - 1)) * 2 + (rem & 1);
    }
#pragma unroll
    for (int q = 0; q < NX; q++) {
        const int idx = min(t + 256 * q, P * KC - 1);
        px[q] = a.in.d + (size_t)(idx / P) * n + min(p0 + idx % P, n - 1);
    }
    const size_t pdo = (size_t)min(r0 / 8 + t / KC, ng - 1) * nb + t % KC, sdo = a.in.s - a.in.d;
    u32x4 ga[NA], gb[NBQ], gd = u32x4{0, 0, 0, 0}, gm = u32x4{0, 0, 0, 0};
    float gxd[NX], gxs[NX];
    auto fetch = [&](int c) {
        const int j0 = c * KC;
#pragma unroll
        for (int q = 0; q < NA; q++) ga[q] = pa[q][j0];
#pragma unroll
        for (int q = 0; q < NBQ; q++) gb[q] = pb[q][(size_t)j0 * n * 2];
        if (t < 8 * KC) {
            gd = ((const u32x4*)a.W.scales)[pdo + j0];
            if (HM) gm = ((const u32x4*)a.W.mins)[pdo + j0];
        }
#pragma unroll
        for (int q = 0; q < NX; q++) {
            gxd[q] = px[q][(size_t)j0 * n];
            gxs[q] = px[q][(size_t)j0 * n + sdo];
        }   // (threads past P * KC re-read the last pair; they store nothing)
    };
    auto stash = [&](int buf) {
#pragma unroll
        for (int q = 0; q < NA; q++) {   // byte k of the record: low nibble of code byte k (k < 16), high of k - 16
            const int idx = t + 256 * q;
            uint2* dst = (uint2*)&sA[buf][(idx / KC) * SA + 8 * (idx % KC)];
            const u32x4 v = ga[q];
            dst[0] = uint2{v.x & 0x0F0F0F0Fu, v.y & 0x0F0F0F0Fu};
            dst[1] = uint2{v.z & 0x0F0F0F0Fu, v.w & 0x0F0F0F0Fu};
            dst[2] = uint2{(v.x >> 4) & 0x0F0F0F0Fu, (v.y >> 4) & 0x0F0F0F0Fu};
            dst[3] = uint2{(v.z >> 4) & 0x0F0F0F0Fu, (v.w >> 4) & 0x0F0F0F0Fu};
        }
#pragma unroll
        for (int q = 0; q < NBQ; q++) {
            const int idx = t + 256 * q, rem = idx % (2 * P);
            sB[buf][idx / (2 * P)][rem >> 1][(rem & 1) ^ ((rem >> 4) & 1)] = gb[q];
        }
        if (t < 8 * KC) {
            const int g = t / KC, jb = t % KC;
            *(u32x4*)&sD[buf][jb][8 * g] = gd;
            if (HM) *(u32x4*)&sM[buf][jb][HM ? 8 * g : 0] = gm;
        }
#pragma unroll
        for (int q = 0; q < NX; q++) {
            const int idx = t + 256 * q;
            if (idx < P * KC) sX[buf][idx / P][idx % P] = float2{gxd[q], gxs[q]};
        }
    };

    // lane l's accumulators: register k = 4 b + i of block b = 2 mt + nt holds row 4 (l / 16) + i of row tile mt
    // at position l % 16 of position tile nt (the layout of both matrix-core results)
    float acc[16];
#pragma unroll
    for (int k = 0; k < 16; k++) acc[k] = 0.0f;
    v16f cor = {0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f};
    const v16f zero = cor;
    // this lane's outer-product operands: row 16 mt + (l % 16) of the wave's rows for block b = l / 16 (mt = b / 2),
    // position 16 nt + (l % 16) of its positions (nt = b % 2; with one position tile, nt = 0 again)
    const int orow = rl + 16 * (lane >> 5) + li, opos = pl + 16 * (NTW == 2 ? (lane >> 4) & 1 : 0) + li;
    const uint64_t et = EPI == EPI_SWIGLU ? kExp2Tab[t & 31] : 0;   // (requested first: its wait needs nothing later)
    fetch(0);
    stash(0);
    if (EPI == EPI_SWIGLU && t < 32) sE[t] = et;
    __syncthreads();
    for (int c = 0; c < nch; c++) {
        const int buf = c & 1;
        if (c + 1 < nch) fetch(c + 1);
        // the narrow tiles (fewer than 2 workgroups per CU) take a whole chunk's blocks in one unrolled body, their
        // LDS reads and matrix-core products all issued ahead of the chains (the register room 2 workgroups per CU allow)
#pragma unroll(PW == 16 ? KC : 2)
        for (int jb = 0; jb < KC; jb++) {
            i32x4 isum[2][NTW];
            long cb[NTW];
#pragma unroll
            for (int nt = 0; nt < NTW; nt++)   // (li & 8: the halves were swapped, which spreads the reads over the banks)
                cb[nt] = ((const long*)&sB[buf][jb][pl + 16 * nt + li][0])[lq ^ ((li >> 3) << 1)];
#pragma unroll
            for (int mt = 0; mt < 2; mt++) {   // columns 8 (lq & 1) .. + 7, low nibbles for lq < 2, else high
                const long av = *(const long*)&sA[buf][(rl + 16 * mt + li) * SA + 8 * jb + 2 * lq];
#pragma unroll
                for (int nt = 0; nt < NTW; nt++)
                    isum[mt][nt] = __builtin_amdgcn_mfma_i32_16x16x32_i8(av, cb[nt], i32x4{0, 0, 0, 0}, 0, 0, 0);
            }
            const float dl = h2f(sD[buf][jb][orow]);
            const float ml = HM ? h2f(sM[buf][jb][HM ? orow : 0]) : dl;
            const float2 xl = sX[buf][jb][opos];
            const v16f dd = __builtin_amdgcn_mfma_f32_16x16x1f32(dl, xl.x, zero, 0, 0, 0);
            cor = __builtin_amdgcn_mfma_f32_16x16x1f32(ml, xl.y, cor, 0, 0, 0);
#pragma unroll
            for (int mt = 0; mt < 2; mt++)
#pragma unroll
                for (int nt = 0; nt < NTW; nt++)
#pragma unroll
                    for (int i = 0; i < 4; i++) {
                        const int k = 4 * (2 * mt + nt) + i;
                        acc[k] = fmaf((float)isum[mt][nt][i], dd[k], acc[k]);
                    }
        }
        if (c + 1 < nch) stash(buf ^ 1);
        __syncthreads();
    }
    const int rbase = r0 + rl, pbase = p0 + pl;
    // EPI_SWIGLU with outc: the workgroup's 64 rows are one 32-channel cut block of the output; its activations are
    // staged in LDS (the code tiles' space, free after the last chunk's barrier), [position][channel], 33 floats apart
    const bool cut_out = EPI == EPI_SWIGLU && a.outc.q != nullptr;
    float* act = reinterpret_cast<float*>(&sA[0][0]);
#pragma unroll
    for (int mt = 0; mt < 2; mt++)
#pragma unroll
        for (int nt = 0; nt < NTW; nt++) {
            const int p = pbase + 16 * nt + li, rr0 = rbase + 16 * mt + 4 * lq;
            float v[4];
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const int k = 4 * (2 * mt + nt) + i;
                v[i] = HM ? acc[k] + cor[k] : fmaf(-8.0f, cor[k], acc[k]);
            }
            if (EPI == EPI_SWIGLU) {
                // rows 0-7 of the 16-row tile are a gate group, rows 8-15 the matching up group (lanes + 32): lane l
                // (lq < 2) forms channels 4 lq, 4 lq + 1 of the tile's 8 and lane l + 32 channels 4 lq + 2, 4 lq + 3,
                // each sending its partner the two values that one needs, so every lane evaluates two activations
                const bool lo = lq < 2;
                const float s0 = __shfl_xor(lo ? v[2] : v[0], 32), s1 = __shfl_xor(lo ? v[3] : v[1], 32);
                const float g0 = lo ? v[0] : s0, g1 = lo ? v[1] : s1, u0 = lo ? s0 : v[2], u1 = lo ? s1 : v[3];
                const int ch = (rl + 16 * mt) / 2 + 4 * (lq & 1) + (lo ? 0 : 2);   // channel within the workgroup's 32
                if (cut_out) {   // to LDS for the block cut below
                    act[(pl + 16 * nt + li) * 33 + ch] = silu_t(g0, sE) * u0;
                    act[(pl + 16 * nt + li) * 33 + ch + 1] = silu_t(g1, sE) * u1;
                } else if (p < n && rbase + 16 * mt < rows) {
                    float* o = a.out + (size_t)p * a.out_ld + r0 / 2 + ch;
                    o[0] = silu_t(g0, sE) * u0;
                    o[1] = silu_t(g1, sE) * u1;
                }
            } else if (p < n) {
                float* o = a.out + (size_t)p * a.out_ld + rr0;
#pragma unroll
                for (int i = 0; i < 4; i++)
                    if (rr0 + i < rows) o[i] = v[i];
            }
        }
    if (EPI == EPI_SWIGLU && cut_out) {
        // the cut of each position's block (imi_cut32's values, as cut_store): thread (position, quarter) holds 8
        // channels; amax and the code sum are order-free reductions, over the quad of lanes by DPP
        static_assert(sizeof(sA) >= (size_t)P * 33 * sizeof(float), "activation staging");
        __syncthreads();
        const int jb = r0 / 64;
        for (int e = t; e < P * 4; e += 256) {   // (P * 4 is 256 or 128: whole waves)
            const int pp = e >> 2, qq = e & 3, p = p0 + pp;
            float x8[8];
#pragma unroll
            for (int k = 0; k < 8; k++) x8[k] = act[pp * 33 + 8 * qq + k];
            float am = 0.0f;
#pragma unroll
            for (int k = 0; k < 8; k++) am = fmaxf(am, fabsf(x8[k]));
            am = fmaxf(am, dppf<DPP_XOR1>(am));
            am = fmaxf(am, dppf<DPP_XOR2>(am));
            const float d = am / 127.0f, id = d != 0.0f ? 1.0f / d : 0.0f;
            unsigned w2[2] = {0u, 0u};
            int sum = 0;
#pragma unroll
            for (int k = 0; k < 8; k++) {
                const int q = (int)rintf(x8[k] * id);
                sum += q;
                w2[k >> 2] |= ((unsigned)q & 0xFFu) << (8 * (k & 3));
            }
            sum += dppi<DPP_XOR1>(sum);
            sum += dppi<DPP_XOR2>(sum);
            if (p < n) {
                *reinterpret_cast<uint2*>(a.outc.q + ((size_t)jb * n + p) * 32 + 8 * qq) = uint2{w2[0], w2[1]};
                if (qq == 0) {
                    a.outc.d[(size_t)jb * n + p] = d;
                    a.outc.s[(size_t)jb * n + p] = d * (float)sum;
                }
            }
        }
    }
}

// ---------------------------------------------------------------- gated short conv along positions
// thread per (position p, channel e): u = c * (b x w_d + taps), the taps being the b x values of the d_conv positions
// before p (from this batch, or the conversation's conv memory before it), fma-chained oldest first
// (imi/core/seoul.cpp:562-577); then the cut of each 32 outputs: the 32 channels of a cut block are 32 lanes, which
// reduce amax and the code sum across lanes (imi_cut32's values; the max and the integer sum do not depend on order)
__global__ __launch_bounds__(256) void k_pf_conv_lanes(pf_conv_args a) {
    const int E = a.E, dc = a.d_conv, gid = blockIdx.x * 256 + threadIdx.x;
    const bool on = gid < a.n * E;
    const int p = on ? gid / E : 0, e = on ? gid - p * E : 0, t = e >> 5, c = e & 31;
    const size_t ld = 3 * (size_t)E;
    const int ub = 96 * t + 24 * (c >> 3) + (c & 7);
    const float* r = a.bcx + (size_t)p * ld + ub;
    float u = 0.0f;
    if (on) {
        const float bx = r[0] * r[16];
        float sv = bx * a.w[(size_t)dc * E + e];
        for (int tt = 0; tt < dc; tt++) {
            const int q = p - dc + tt;
            float st;
            if (q >= 0) {
                const float* rq = a.bcx + (size_t)q * ld + ub;
                st = rq[0] * rq[16];
            } else {
                st = a.state[(size_t)(p + tt) * E + e];
            }
            sv = fmaf(st, a.w[(size_t)tt * E + e], sv);
        }
        u = sv * r[8];
    }
    float amax = fabsf(u);
#pragma unroll
    for (int o = 16; o > 0; o >>= 1) amax = fmaxf(amax, __shfl_xor(amax, o));
    const float d = amax / 127.0f, id = d != 0.0f ? 1.0f / d : 0.0f;
    const int q = (int)rintf(u * id);
    int sum = q;
#pragma unroll
    for (int o = 16; o > 0; o >>= 1) sum += __shfl_xor(sum, o);
    if (on) {
        a.cut.q[((size_t)t * a.n + p) * 32 + c] = (int8_t)q;
        if (c == 0) {
            a.cut.d[(size_t)t * a.n + p] = d;
            a.cut.s[(size_t)t * a.n + p] = d * (float)sum;
        }
    }
}

// the conv memory after the batch: its last d_conv b x values (older memory where the batch is shorter)

// ---------------------------------------------------------------- attention
// keys and values of the batch into the fp16 cache: k = rope(norm(k) * k_norm) at the position (imi/core/seoul.cpp:
// 590-601); one wave per (position, kv head)
__global__ __launch_bounds__(64) void k_pf_kv(pf_attn_args a) {
    __shared__ float st[128];
    const int p = blockIdx.x, g = blockIdx.y, lane = threadIdx.x, D = a.D;
    const int at = a.pos0 + p, Hq = a.n_head * D, kvd = a.n_kv * D;
    const float* row = a.qkv + (size_t)p * a.ld;
    float kd[2];
    const float2* cs = a.rope_cs + (size_t)at * (D / 2);
    if (D > 64) head_norm_rope<2>(row + Hq + g * D, a.k_norm, (float*)st, cs, D, a.eps, kd);
    else head_norm_rope<1>(row + Hq + g * D, a.k_norm, (float*)st, cs, D, a.eps, kd);
    for (int c = 0; c < 2; c++) {
        const int e = lane + 64 * c;
        if (e < D) {
            a.kc[((size_t)g * a.n_ctx + at) * D + e] = f2h(kd[c]);
            a.vc[((size_t)g * a.n_ctx + at) * D + e] = f2h(row[Hq + kvd + g * D + e]);
        }
    }
}

// workgroup per (position, kv head), its query heads together (imi/core/seoul.cpp:602-621): q = rope(norm(q) *
// q_norm); score_t = dot_h(q, K_t) / sqrt(D) over the causal window; softmax with the max subtracted, glibc's expf and
// a double sum in position order; o = sum_t fma(e_t * inv, V_t, o) in order; times the sigmoid head gate; the
// output rows cut per 32 channels for the o table
// lowest set bit exponent of a positive float (0 gives a large value)
__device__ __forceinline__ int low_bit_exp(float e) {
    const unsigned b = __float_as_uint(e), ex = b >> 23, mt = b & 0x7FFFFFu;
    if (b == 0) return 1 << 20;
    return ex == 0 ? -149 + __builtin_ctz(mt) : (int)ex - 150 + __builtin_ctz(mt | 0x800000u);
}

template <int D>
__global__ __launch_bounds__(256) void k_pf_attn(pf_attn_args a) {
    extern __shared__ float lds[];
    const int p = blockIdx.x, g = blockIdx.y, tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    constexpr int half = D / 2;
    const int Hq = a.n_head * D, kvd = a.n_kv * D, grp = a.n_head / a.n_kv;
    const int at = a.pos0 + p;
    const int s0 = a.n_swa > 0 ? max(0, at - a.n_swa + 1) : 0, nk = at - s0 + 1, nks = a.pos0 + a.n;
    const uint16_t* kc = a.kc + (size_t)g * a.n_ctx * D;
    const uint16_t* vc = a.vc + (size_t)g * a.n_ctx * D;
    const float* row = a.qkv + (size_t)p * a.ld;
    float* q_s = lds;                      // [grp][D]
    float* o_s = q_s + grp * D;            // [grp][D]
    float* scratch = o_s + grp * D;        // [4][D]
    float* inv_s = scratch + 4 * D;        // [8]
    float* sc = inv_s + 8;                 // [grp][nks]
    const float2* cs = a.rope_cs + (size_t)at * half;

    constexpr int DPL = (D + 63) / 64;
    for (int hh = wv; hh < grp; hh += 4) {
        float r[DPL];
        head_norm_rope<DPL>(row + (g * grp + hh) * D, a.q_norm, scratch + wv * D, cs, D, a.eps, r);
#pragma unroll
        for (int c = 0; c < DPL; c++)
            if (lane + 64 * c < D) q_s[hh * D + lane + 64 * c] = r[c];
    }
    __syncthreads();

    const float scale = 1.0f / sqrtf((float)D);
    for (int t = tid; t < nk; t += 256) {
        const uint16_t* kt = kc + (size_t)(s0 + t) * D;
        float kf[D];
#pragma unroll
        for (int i0 = 0; i0 < D; i0 += 8) {
            const u32x4 kw = *reinterpret_cast<const u32x4*>(kt + i0);
            const unsigned w4[4] = {kw.x, kw.y, kw.z, kw.w};
#pragma unroll
            for (int e = 0; e < 8; e++) kf[i0 + e] = h2f((uint16_t)((w4[e >> 1] >> (16 * (e & 1))) & 0xFFFFu));
        }
        for (int hh = 0; hh < grp; hh++) sc[(size_t)hh * nks + t] = dot_h8<D>(q_s + hh * D, kf) * scale;
    }
    __syncthreads();
    // softmax per head (wave hh): max, e_t = glibc expf(s_t - max), the double sum of e_t in position order (its
    // exact-sum shortcut: when every e_t is a multiple of 2^(B - 51), B = floor(log2 sum), any order gives the same
    // double, so the wave's tree sum is used; otherwise lane 0 adds in order), then a_t = e_t * inv in place
    for (int hh = wv; hh < grp; hh += 4) {
        float* s = sc + (size_t)hh * nks;
        float mx = -INFINITY;
        for (int t = lane; t < nk; t += 64) mx = fmaxf(mx, s[t]);
        mx = wave_max(mx);
        double part = 0.0;
        int lowb = 1 << 20;
        for (int t = lane; t < nk; t += 64) {
            const float e = expf_glibc(s[t] - mx);
            s[t] = e;
            part += (double)e;
            lowb = min(lowb, low_bit_exp(e));
        }
#pragma unroll
        for (int o = 32; o > 0; o >>= 1) {
            part += __shfl_xor(part, o);
            lowb = min(lowb, __shfl_xor(lowb, o));
        }
        __builtin_amdgcn_wave_barrier();
        float inv = 0.0f;
        if (lane == 0) {
            int ex;
            (void)frexp(part, &ex);
            if (lowb < ex - 1 - 51) {   // some e_t below the exact unit: add in position order, as imi's loop
                double sum = 0.0;
                for (int t = 0; t < nk; t++) sum += (double)s[t];
                part = sum;
            }
            inv = (float)(1.0 / part);
        }
        inv = __shfl(inv, 0);
        for (int t = lane; t < nk; t += 64) s[t] = s[t] * inv;
    }
    __syncthreads();
    // o = sum_t fma(a_t, V_t, o) in position order, thread per (head, dimension); value rows staged through LDS in
    // tiles of TP positions, shared by the group's heads
    constexpr int TP = 32, TW = TP * D / 8;   // positions per tile, 16-byte words per tile
    u32x4* vt = (u32x4*)(sc + (size_t)grp * ((nks + 3) & ~3));
    const uint16_t* vh = (const uint16_t*)vt;
    const int nitem = grp * D;                // (head, dimension) items, at most 4 per thread
    float o[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    // a tile is TP * D / 8 16-byte words (at most 512: 2 per thread); the next tile's words are requested before the
    // current tile's chains run
    constexpr int WPT = (TW + 255) / 256;
    u32x4 nv[WPT];
    auto fetch = [&](int q0) {
        const int nt = min(TP, nk - q0);
#pragma unroll
        for (int r = 0; r < WPT; r++) {
            const int w = tid + 256 * r;
            if (w < nt * (D / 8)) nv[r] = ((const u32x4*)(vc + (size_t)(s0 + q0) * D))[w];
        }
    };
    fetch(0);
    for (int q0 = 0; q0 < nk; q0 += TP) {
        const int nt = min(TP, nk - q0);
        __syncthreads();
#pragma unroll
        for (int r = 0; r < WPT; r++) {
            const int w = tid + 256 * r;
            if (w < nt * (D / 8)) vt[w] = nv[r];
        }
        __syncthreads();
        if (q0 + TP < nk) fetch(q0 + TP);
#pragma unroll
        for (int c = 0; c < 4; c++) {
            const int k = tid + 256 * c;
            if (k < nitem) {
                const int hh = k / D, i = k - hh * D;
                const float* av = sc + (size_t)hh * nks + q0;
                float acc = o[c];
                if (nt == TP) {   // a full tile: every operand requested before the chain runs
                    float aa[TP], vv[TP];
#pragma unroll
                    for (int t = 0; t < TP; t++) {
                        aa[t] = av[t];
                        vv[t] = h2f(vh[t * D + i]);
                    }
#pragma unroll
                    for (int t = 0; t < TP; t++) acc = fmaf(aa[t], vv[t], acc);
                } else {
                    for (int t = 0; t < nt; t++) acc = fmaf(av[t], h2f(vh[t * D + i]), acc);
                }
                o[c] = acc;
            }
        }
    }
#pragma unroll
    for (int c = 0; c < 4; c++) {
        const int k = tid + 256 * c;
        if (k < nitem) {
            const int hh = k / D, h = g * grp + hh;
            const float gate = 1.0f / (1.0f + expf_glibc(-row[Hq + 2 * kvd + h]));
            o_s[k] = o[c] * gate;
        }
    }
    __syncthreads();
    const int nblk = grp * D / 32, cb0 = g * nblk;
    if (tid < nblk) cut_store(a.cut, a.n, cb0 + tid, p, o_s + 32 * tid);
}

// The same attention with its products on the matrix cores, for groups of at most 4 query heads per kv head: a
// workgroup takes 4 consecutive positions of one kv head (the last positions, with the most keys, first), their
// 4 x 4 (position, head) pairs being 16 rows R = 4 (position) + (head) (head slots past the group are zero and
// dropped). The fp32 K = 1 matrix ops used round once, like fmaf, and equal the VALU's fmaf bit for bit (the prefill
// tables run their scale chains on them).
// Scores, v_mfma_f32_16x16x1_4b_f32 (lane l supplies row l % 16 of block l / 16 (A) and column l % 16 of block l / 16
// (B); register 4 b + i of lane l holds block b's row 4 (l / 16) + i, column l % 16): dot_h's 8 chains (chain j over
// dimensions j, j + 8, ...), 16 keys per tile, block b holding chain 2 b (one instruction) and 2 b + 1 (the other)
// at each step m, so lane l takes key l % 16 and the fp16 pair at dimensions 8 m + 2 (l / 16), + 1 (the 4 lanes of a
// key read consecutive words of its row), and every chain of a (row, key) ends in one lane: ((a0 + a4) + (a2 + a6)) +
// ((a1 + a5) + (a3 + a7)) runs in registers. Every key of the 4 positions' union is scored; each row's softmax reads
// its own range. Values: o = fma(a_t, V_t, o) over each position's keys in order, a wave per position (below).
template <int D>
__global__ __launch_bounds__(256) void k_pf_attn_mf(pf_attn_args a) {
    typedef float v16f __attribute__((ext_vector_type(16)));
    extern __shared__ float lds[];
    constexpr int NM = D / 8, DPL = (D + 63) / 64, NWV = (D + 63) / 64, CH = 8, TPV = 64, VPT = TPV * D / 8 / 256;
    constexpr int KR = D > 64 ? 2 : 4;   // key tiles in flight per wave
    const int tid = threadIdx.x, lane = tid & 63, wv = __builtin_amdgcn_readfirstlane(tid >> 6), g = blockIdx.y;
    const int grp = a.n_head / a.n_kv, Hq = a.n_head * D, kvd = a.n_kv * D;
    // the longest key ranges (last positions) first
    const int p0 = 4 * ((int)gridDim.x - 1 - (int)blockIdx.x), plast = min(p0 + 3, a.n - 1);
    auto win0 = [&](int at) { return a.n_swa > 0 ? max(0, at - a.n_swa + 1) : 0; };
    // (score rows 4 floats past a multiple of 32 apart: a wave's 4 rows of one key in distinct LDS banks)
    const int sU = win0(a.pos0 + p0), nkU = a.pos0 + plast - sU + 1, ldk = ((nkU + 31) & ~31) + 4;
    const uint16_t* kc = a.kc + ((size_t)g * a.n_ctx + sU) * D;
    const uint16_t* vc = a.vc + ((size_t)g * a.n_ctx + sU) * D;
    uint64_t* etab = (uint64_t*)lds;   // expf's table (a copy in LDS: no memory round trip inside the softmax)
    float* q_s = lds + 64;             // [16][D] query rows, later the gated outputs [4][grp * D]
    float* gate_s = q_s + 16 * D;      // [16]
    float* sc = gate_s + 16;           // [16][ldk] scores, then weights; the rows' norm staging before the scores
    u32x4* vt_s = (u32x4*)(sc + 16 * ldk + 4 * D);   // 2 value tiles [TPV][D] fp16
    const float scale = 1.0f / sqrtf((float)D);
    // wave w makes and normalises rows w + 4 k (head w of position k, a head slot past the group being zero)
    const bool hv = wv < grp;
    const int hq = min(wv, grp - 1);
    int r0[4], r1[4];   // row k's keys (union-relative)
#pragma unroll
    for (int k = 0; k < 4; k++) {
        const int at = a.pos0 + min(p0 + k, a.n - 1);
        r0[k] = win0(at) - sU;
        r1[k] = at - sU;
    }

    const uint64_t et = kExp2Tab[tid & 31];
    const float gin = a.qkv[(size_t)min(p0 + ((tid >> 2) & 3), a.n - 1) * a.ld + Hq + 2 * kvd + g * grp +
                            min(tid & 3, grp - 1)];   // (threads 0-15: the head gates' inputs)
    // this wave's key tiles (tile tt = wv + 4 it covers keys 16 tt ..), then its 4 query rows' operands
    const int ntile = (nkU + 15) >> 4, nit = ntile > wv ? (ntile - wv + 3) >> 2 : 0;
    const int cb = lane >> 4, kk = lane & 15;
    unsigned kw[KR][NM];
    auto kload = [&](unsigned (&w)[NM], int it) {
        const unsigned* kr = (const unsigned*)(kc + (size_t)min(16 * (wv + 4 * it) + kk, nkU - 1) * D) + cb;
#pragma unroll
        for (int m = 0; m < NM; m++) w[m] = kr[4 * m];
    };
#pragma unroll
    for (int r = 0; r < KR; r++) kload(kw[r], r);
    {
        float xq[4][DPL], wq[DPL];
        float2 cz[4][DPL];
#pragma unroll
        for (int k = 0; k < 4; k++) {
            const int pr = min(p0 + k, a.n - 1);
            norm_rope_load<DPL>(a.qkv + (size_t)pr * a.ld + (g * grp + hq) * D, a.q_norm,
                                a.rope_cs + (size_t)(a.pos0 + pr) * (D / 2), D, xq[k], wq, cz[k]);
        }
#pragma unroll
        for (int k = 0; k < 4; k++) {
            float r[DPL];
            norm_rope_vals<DPL>(xq[k], wq, sc + wv * D, cz[k], D, a.eps, r);
#pragma unroll
            for (int c = 0; c < DPL; c++)
                if (lane + 64 * c < D) q_s[(wv + 4 * k) * D + lane + 64 * c] = hv ? r[c] : 0.0f;
        }
    }
    if (tid < 32) etab[tid] = et;
    __syncthreads();

    // scores of 16 rows x 16 keys per tile
    {
        float qa[NM], qb[NM];
#pragma unroll
        for (int m = 0; m < NM; m++) {
            const float2 v = *(const float2*)&q_s[kk * D + 8 * m + 2 * cb];
            qa[m] = v.x;
            qb[m] = v.y;
        }
        auto tile = [&](const unsigned (&w)[NM], int it) {
            v16f lo, hi;
#pragma unroll
            for (int k = 0; k < 16; k++) lo[k] = hi[k] = 0.0f;
#pragma unroll
            for (int m = 0; m < NM; m++) {
                lo = __builtin_amdgcn_mfma_f32_16x16x1f32(qa[m], h2f((uint16_t)(w[m] & 0xFFFFu)), lo, 0, 0, 0);
                hi = __builtin_amdgcn_mfma_f32_16x16x1f32(qb[m], h2f((uint16_t)(w[m] >> 16)), hi, 0, 0, 0);
            }
            const int t = 16 * (wv + 4 * it) + kk;
            if (t < nkU) {
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    const float s = ((lo[i] + lo[8 + i]) + (lo[4 + i] + lo[12 + i])) +
                                    ((hi[i] + hi[8 + i]) + (hi[4 + i] + hi[12 + i]));
                    sc[(4 * cb + i) * ldk + t] = s * scale;
                }
            }
        };
        for (int it0 = 0; it0 < nit; it0 += KR) {
#pragma unroll
            for (int r = 0; r < KR; r++) {
                if (it0 + r < nit) tile(kw[r], it0 + r);
                kload(kw[r], it0 + r + KR);   // (past the wave's tiles: the last key's row again, a cache hit)
            }
        }
    }
    __syncthreads();

    // values stream through LDS in tiles of TPV keys over the union, fetched by every thread two tiles ahead (16-byte
    // words into registers, then stored to the tile's buffer); the first two tiles are requested before the softmax
    const int ntv = (nkU + TPV - 1) / TPV;
    u32x4 vw[2][VPT];
    auto vfetch = [&](u32x4 (&w)[VPT], int i) {
#pragma unroll
        for (int r = 0; r < VPT; r++) {
            const int q = tid + 256 * r, t = min(TPV * i + q / (D / 8), nkU - 1);
            w[r] = ((const u32x4*)(vc + (size_t)t * D))[q % (D / 8)];
        }
    };
    vfetch(vw[0], 0);
    vfetch(vw[1], 1);

    // softmax per row over its own keys: max, e_t = glibc expf(s_t - max), the double sum of e_t in position order
    // (its exact-sum shortcut: when every e_t is a multiple of 2^(B - 51), B = floor(log2 sum), any order gives the
    // same double, so the wave's tree sum is used), then a_t = e_t * inv in place. The wave's 4 rows run side by
    // side (their ranges differ by at most 3 keys at either end); the in-order sums of the rows that need them run
    // side by side in lanes 0-3, 8 keys' values read ahead of their adds.
    if (tid < 16) gate_s[tid] = 1.0f / (1.0f + expf_glibc_t(-gin, etab));   // head gates
    float* sw = sc + (size_t)wv * ldk;   // row k of this wave at sw + 4 k ldk
    double wpart[4] = {1.0, 1.0, 1.0, 1.0};
    int wlow[4] = {1 << 20, 1 << 20, 1 << 20, 1 << 20};
    if (hv) {
        float mx[4] = {-INFINITY, -INFINITY, -INFINITY, -INFINITY};
        for (int t = r0[0] + lane; t <= r1[3]; t += 64) {
#pragma unroll
            for (int k = 0; k < 4; k++)
                if (t >= r0[k] && t <= r1[k]) mx[k] = fmaxf(mx[k], sw[4 * k * ldk + t]);
        }
#pragma unroll
        for (int k = 0; k < 4; k++) {
            mx[k] = wave_max(mx[k]);
            wpart[k] = 0.0;
        }
        for (int t = r0[0] + lane; t <= r1[3]; t += 64) {
#pragma unroll
            for (int k = 0; k < 4; k++)
                if (t >= r0[k] && t <= r1[k]) {
                    const float e = expf_glibc_t(sw[4 * k * ldk + t] - mx[k], etab);
                    sw[4 * k * ldk + t] = e;
                    wpart[k] += (double)e;
                    wlow[k] = min(wlow[k], low_bit_exp(e));
                }
        }
#pragma unroll
        for (int k = 0; k < 4; k++)
#pragma unroll
            for (int o = 32; o > 0; o >>= 1) {
                wpart[k] += __shfl_xor(wpart[k], o);
                wlow[k] = min(wlow[k], __shfl_xor(wlow[k], o));
            }
    }
    __builtin_amdgcn_wave_barrier();
    float inv = 0.0f;
    if (lane < 4 && hv) {
        double part = wpart[0];
        int lowb = wlow[0], q0 = r0[0], q1 = r1[0];
#pragma unroll
        for (int k = 1; k < 4; k++)
            if (lane == k) {
                part = wpart[k];
                lowb = wlow[k];
                q0 = r0[k];
                q1 = r1[k];
            }
        int ex;
        (void)frexp(part, &ex);
        if (lowb < ex - 1 - 51) {   // some e_t below the exact unit: add in position order, as imi's loop
            const float* s = sw + (size_t)4 * lane * ldk;
            double sum = 0.0;
            int t = q0;
            for (; t + 8 <= q1 + 1; t += 8) {
                float v[8];
#pragma unroll
                for (int j = 0; j < 8; j++) v[j] = s[t + j];
#pragma unroll
                for (int j = 0; j < 8; j++) sum += (double)v[j];
            }
            for (; t <= q1; t++) sum += (double)s[t];
            part = sum;
        }
        inv = (float)(1.0 / part);
    }
    {
        float ik[4];
#pragma unroll
        for (int k = 0; k < 4; k++) ik[k] = __shfl(inv, k);
        if (hv)
            for (int t = r0[0] + lane; t <= r1[3]; t += 64) {
#pragma unroll
                for (int k = 0; k < 4; k++)
                    if (t >= r0[k] && t <= r1[k]) sw[4 * k * ldk + t] = sw[4 * k * ldk + t] * ik[k];
            }
    }
    __syncthreads();

    // values: wave w runs position w's chains over its own keys in order, v_mfma_f32_4x4x1_16b_f32 (d[l][i] =
    // fma(a[4 (l / 4) + i], b[l], c[l][i]), one rounding, bit for bit fmaf): lane l supplies head l % 4's weight and
    // the value of dimension l (of each 64), and holds head i's output of dimension l in register i; a chunk of CH
    // keys at either end of the wave's range takes the keys outside it as a zero weight times a zero value (o + 0 =
    // o: o starts at +0 and so never becomes -0)
    typedef float v4f __attribute__((ext_vector_type(4)));
    v4f o[NWV];
#pragma unroll
    for (int c = 0; c < NWV; c++) o[c] = v4f{0.0f, 0.0f, 0.0f, 0.0f};
    const int w0 = r0[wv], w1 = r1[wv];
    const float* aw = sc + (size_t)(4 * wv + (lane & 3)) * ldk;
    // (two tiles per pass, so that each register set is named at compile time; a pass past the last tile stores and
    // fetches clamped rows that nothing reads)
    for (int i0 = 0; i0 < ntv; i0 += 2) {
#pragma unroll
        for (int h = 0; h < 2; h++) {
            const int i = i0 + h;
            u32x4* vb = vt_s + (size_t)h * (TPV * D / 8);
            const uint16_t* vh = (const uint16_t*)vb;
#pragma unroll
            for (int r = 0; r < VPT; r++) vb[tid + 256 * r] = vw[h][r];
            __syncthreads();
            vfetch(vw[h], i + 2);
            if (i < ntv) {
#pragma unroll
                for (int c = 0; c < TPV / CH; c++) {
                    const int tb = TPV * i + CH * c;
                    if (tb + CH - 1 < w0 || tb > w1) continue;
                    const bool full = tb >= w0 && tb + CH - 1 <= w1;
                    const float4 a0 = *(const float4*)(aw + tb), a1 = *(const float4*)(aw + tb + 4);
                    const float av[CH] = {a0.x, a0.y, a0.z, a0.w, a1.x, a1.y, a1.z, a1.w};
                    unsigned vv[NWV][CH];
#pragma unroll
                    for (int j = 0; j < CH; j++)
#pragma unroll
                        for (int cc = 0; cc < NWV; cc++) vv[cc][j] = vh[(CH * c + j) * D + min(64 * cc + lane, D - 1)];
#pragma unroll
                    for (int j = 0; j < CH; j++) {
                        const bool in = full || (tb + j >= w0 && tb + j <= w1);
#pragma unroll
                        for (int cc = 0; cc < NWV; cc++)
                            o[cc] = __builtin_amdgcn_mfma_f32_4x4x1f32(in ? av[j] : 0.0f, in ? h2f((uint16_t)vv[cc][j]) : 0.0f,
                                                                       o[cc], 0, 0, 0);
                    }
                }
            }
        }
    }
    // gated outputs, position-major [4][grp * D] in q_s (free since the scores)
#pragma unroll
    for (int cc = 0; cc < NWV; cc++) {
        const int d = 64 * cc + lane;
#pragma unroll
        for (int i = 0; i < 4; i++)
            if (i < grp && d < D) q_s[(wv * grp + i) * D + d] = o[cc][i] * gate_s[4 * wv + i];
    }
    __syncthreads();
    const int nblk = grp * D / 32, cb0 = g * nblk;
    for (int k = tid; k < 4 * nblk; k += 256) {
        const int pq = k / nblk, j = k - pq * nblk;
        if (p0 + pq < a.n) cut_store(a.cut, a.n, cb0 + j, p0 + pq, q_s + pq * grp * D + 32 * j);
    }
}

}  // namespace

hipError_t launch_pf_rows(int mode, const pf_rows_args& a, hipStream_t s) {
    if (a.E % 32 || a.E > 2048 || a.n < 1) return hipErrorInvalidValue;
    const int extra = mode == PFR_RESID && a.conv.state ? (a.conv.E + 64 * PFR_PPW - 1) / (64 * PFR_PPW) : 0;
    if (extra && (a.conv.E % 32 || a.conv.n < 1 || a.conv.d_conv < 1 || !a.conv.bcx)) return hipErrorInvalidValue;
    const dim3 grid((unsigned)((a.n + PFR_PPW - 1) / PFR_PPW + extra));
    if (mode == PFR_FIRST)
        hipLaunchKernelGGL(k_pf_rows<PFR_FIRST>, grid, dim3(64 * PFR_PPW), 0, s, a);
    else
        hipLaunchKernelGGL(k_pf_rows<PFR_RESID>, grid, dim3(64 * PFR_PPW), 0, s, a);
    return hipGetLastError();
}

#ifndef PF_KC
#define PF_KC 4   // blocks staged per step of the LDS-staged product
#endif
// SEOUL_HIP_PF_PLAIN=1 keeps the products on the unstaged kernel (a comparison switch)
static bool getenv_pf_plain() {
    static const int v = [] { const char* e = getenv("SEOUL_HIP_PF_PLAIN"); return e && e[0] == '1' ? 1 : 0; }();
    return v != 0;
}

bool pf_swiglu_cut_takes(const pf_gemm_args& a) {
    return a.n >= 1 && a.W.rows % 64 == 0 && a.out_ld * 2 == a.W.rows && a.W.nb % PF_KC == 0 && !getenv_pf_plain();
}

hipError_t launch_pf_gemm(int epi, const pf_gemm_args& a, hipStream_t s) {
    if (a.n < 1 || a.W.rows % 8 || (epi == EPI_SWIGLU && a.W.rows % 16)) return hipErrorInvalidValue;
    if (a.outc.q && (epi != EPI_SWIGLU || !a.outc.d || !a.outc.s || !pf_swiglu_cut_takes(a))) return hipErrorInvalidValue;
    const dim3 grid((a.W.rows + 63) / 64, (a.n + 63) / 64);
    const bool hm = a.W.mins != nullptr;   // Q4_1 table
    if (a.W.nb % PF_KC == 0 && !getenv_pf_plain()) {
        // 16 positions per wave when 32 would leave fewer than two waves per SIMD
        const bool narrow = (size_t)grid.x * grid.y * 4 < 2048;
        const dim3 g16(grid.x, (a.n + 31) / 32);
#define SH_PF_LDS(EPI_, HM_)                                                                                      \
    if (narrow) hipLaunchKernelGGL((k_pf_gemm_lds<EPI_, HM_, PF_KC, 16>), g16, dim3(256), 0, s, a);            \
    else hipLaunchKernelGGL((k_pf_gemm_lds<EPI_, HM_, PF_KC, 32>), grid, dim3(256), 0, s, a);
        if (epi == EPI_SWIGLU && hm) { SH_PF_LDS(EPI_SWIGLU, true) }
        else if (epi == EPI_SWIGLU) { SH_PF_LDS(EPI_SWIGLU, false) }
        else if (epi == EPI_STORE && hm) { SH_PF_LDS(EPI_STORE, true) }
        else if (epi == EPI_STORE) { SH_PF_LDS(EPI_STORE, false) }
        else return hipErrorInvalidValue;
#undef SH_PF_LDS
        return hipGetLastError();
    }
    if (epi == EPI_SWIGLU && hm)
        hipLaunchKernelGGL((k_pf_gemm<EPI_SWIGLU, true>), grid, dim3(256), 0, s, a);
    else if (epi == EPI_SWIGLU)
        hipLaunchKernelGGL((k_pf_gemm<EPI_SWIGLU, false>), grid, dim3(256), 0, s, a);
    else if (epi == EPI_STORE && hm)
        hipLaunchKernelGGL((k_pf_gemm<EPI_STORE, true>), grid, dim3(256), 0, s, a);
    else if (epi == EPI_STORE)
        hipLaunchKernelGGL((k_pf_gemm<EPI_STORE, false>), grid, dim3(256), 0, s, a);
    else
        return hipErrorInvalidValue;
    return hipGetLastError();
}

hipError_t launch_pf_cut(const pf_cutk_args& a, hipStream_t s) {
    if (a.K % 32 || a.n < 1) return hipErrorInvalidValue;
    const int total = a.n * (a.K / 32);
    hipLaunchKernelGGL(k_pf_cut, dim3((total + 255) / 256), dim3(256), 0, s, a);
    return hipGetLastError();
}

hipError_t launch_pf_conv_lanes(const pf_conv_args& a, hipStream_t s) {
    if (a.E % 32 || a.n < 1 || a.d_conv < 1) return hipErrorInvalidValue;
    const long long total = (long long)a.n * a.E;   // a thread per (position, channel)
    hipLaunchKernelGGL(k_pf_conv_lanes, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, s, a);
    return hipGetLastError();
}


hipError_t launch_pf_kv(const pf_attn_args& a, hipStream_t s) {
    if (a.D > 128 || a.D % 32 || a.n < 1) return hipErrorInvalidValue;
    hipLaunchKernelGGL(k_pf_kv, dim3(a.n, a.n_kv), dim3(64), 0, s, a);
    return hipGetLastError();
}

// LDS of the prefill attention over `ctx` key positions: the group's query rows, staging, one score row per query
// head of the group and one value tile of 32 positions
static size_t pf_attn_lds(int grp, int D, int ctx) {
    return sizeof(float) * ((size_t)2 * grp * D + 4 * (size_t)D + 8 + (size_t)grp * (((size_t)ctx + 3) & ~(size_t)3)) +
           32 * (size_t)D * sizeof(uint16_t);
}

int pf_attn_max_ctx(int grp, int D) {
    int lo = 0, hi = 1 << 20;
    while (lo < hi) {
        const int mid = (lo + hi + 1) / 2;
        if (pf_attn_lds(grp, D, mid) <= 160 * 1024) lo = mid;
        else hi = mid - 1;
    }
    return lo;
}

// LDS of the matrix-core attention: expf's table, 16 query rows (then the gated outputs), 16 gates, 16 score rows over the
// widest key union of the launch and the 4 rows' norm staging past them, two value tiles of 64 keys
static size_t pf_attn_mf_lds(const pf_attn_args& a) {
    const int nku = a.n_swa > 0 ? std::min(a.pos0 + a.n, a.n_swa + 3) : a.pos0 + a.n, ldk = ((nku + 31) & ~31) + 4;
    return sizeof(float) * (64 + (size_t)16 * a.D + 16 + (size_t)16 * ldk + 4 * (size_t)a.D) + 2 * 64 * (size_t)a.D * 2;
}

hipError_t launch_pf_attn(const pf_attn_args& a, hipStream_t s) {
    const int grp = a.n_head / a.n_kv;
    if (a.n < 1 || a.n_head % a.n_kv) return hipErrorInvalidValue;
    // the matrix-core form for groups of at most 4 heads (SEOUL_HIP_PF_ATTN_VALU=1 keeps the VALU form: a comparison
    // switch, read per launch)
    const char* ev = getenv("SEOUL_HIP_PF_ATTN_VALU");
    const size_t mlds = pf_attn_mf_lds(a);
    if (grp <= 4 && mlds <= 160 * 1024 && !(ev && ev[0] == '1')) {
        const void* fn = a.D == 128 ? (const void*)k_pf_attn_mf<128> : a.D == 64 ? (const void*)k_pf_attn_mf<64>
                       : a.D == 32 ? (const void*)k_pf_attn_mf<32> : nullptr;
        if (fn) {
            if (mlds > 64 * 1024) {
                const hipError_t e = hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, (int)mlds);
                if (e != hipSuccess) return e;
            }
            pf_attn_args b = a;
            void* args[] = {&b};
            return hipLaunchKernel(fn, dim3((a.n + 3) / 4, a.n_kv), dim3(256), args, mlds, s);
        }
    }
    const size_t lds = pf_attn_lds(grp, a.D, a.pos0 + a.n);
    if (lds > 160 * 1024) return hipErrorInvalidValue;
    const void* fn = a.D == 128 ? (const void*)k_pf_attn<128> : a.D == 64 ? (const void*)k_pf_attn<64>
                   : a.D == 32 ? (const void*)k_pf_attn<32> : nullptr;
    if (!fn) return hipErrorInvalidValue;
    if (lds > 64 * 1024) {
        const hipError_t e = hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
        if (e != hipSuccess) return e;
    }
    pf_attn_args b = a;
    void* args[] = {&b};
    return hipLaunchKernel(fn, dim3(a.n, a.n_kv), dim3(256), args, lds, s);
}

}  // namespace sh
