// Device-side helpers shared by the HIP kernels of libseoul_hip (gfx950, wave64).
#pragma once
#include <hip/hip_runtime.h>
#include <hip/hip_fp16.h>
#include <cstdint>

namespace sh {

typedef unsigned u32x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr int WAVE = 64;

// fp16 <-> fp32: v_cvt_f32_f16 is exact (fp16 subnormals are kept: denorm mode 3); fp32 -> fp16 rounds to nearest
// even, as F16C's _cvtss_sh(f, 0) does on the CPU side
__device__ __forceinline__ float h2f(uint16_t h) { return __half2float(__ushort_as_half(h)); }
__device__ __forceinline__ uint16_t f2h(float f) { return __half_as_ushort(__float2half_rn(f)); }

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o);
    return v;
}
__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o));
    return v;
}
__device__ __forceinline__ int wave_isum(int v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o);
    return v;
}

// Q4_0 block dot against an int8-cut input block. Codes are the 16 file bytes (byte i = column i in the low nibble,
// column 16 + i in the high nibble); the input block is 8 dwords of int8 (columns 0..31). Codes 0..15 are valid
// signed bytes, so the signed 4-way dot applies directly; the -8 offset is folded in by the caller.
// Q6_K word table in its tiled device layout (codes: 13 16-byte words per unit, word-major within tiles of 64 units;
// d: fp16 per unit), values 32 j .. 32 j + 31 of a row: block i = j / 8 and 32-value chunk c = j % 8 = 4 h + k of it;
// value l = (low nibble of ql[64 h + 32 (k & 1) + l] for k < 2, high nibble for k >= 2) | (bits 2k, 2k+1 of
// qh[32 h + l]) << 4, and y = (d * scale[8 h + 2 k + l / 16]) * (value - 32) (imi/core/tables.cpp:216-233)
__device__ __forceinline__ void q6k_dequant32(const u32x4* codes, const uint16_t* dv, int nbk, int row, int j, float* v) {
    const int i = j >> 3, c = j & 7, h = c >> 2, k = c & 3;
    const size_t u = (size_t)row * nbk + i;
    const u32x4* base = codes + (u >> 6) * 13 * 64 + (u & 63);
    const int wl = 4 * h + 2 * (k & 1), wh = 8 + 2 * h;
    const u32x4 l0 = base[(size_t)wl * 64], l1 = base[(size_t)(wl + 1) * 64];
    const u32x4 q0 = base[(size_t)wh * 64], q1 = base[(size_t)(wh + 1) * 64];
    const u32x4 sw = base[12 * 64];
    const float d = h2f(dv[u]);
    const unsigned lw[8] = {l0.x, l0.y, l0.z, l0.w, l1.x, l1.y, l1.z, l1.w};
    const unsigned hw[8] = {q0.x, q0.y, q0.z, q0.w, q1.x, q1.y, q1.z, q1.w};
    const unsigned scw[4] = {sw.x, sw.y, sw.z, sw.w};
    const int s0 = 8 * h + 2 * k;
    const float ds0 = d * (float)(int8_t)((scw[s0 >> 2] >> (8 * (s0 & 3))) & 0xFFu);
    const float ds1 = d * (float)(int8_t)((scw[(s0 + 1) >> 2] >> (8 * ((s0 + 1) & 3))) & 0xFFu);
#pragma unroll
    for (int l = 0; l < 32; l++) {
        const unsigned lb = (lw[l >> 2] >> (8 * (l & 3))) & 0xFFu, hb = (hw[l >> 2] >> (8 * (l & 3))) & 0xFFu;
        const int q = (int)(((k < 2 ? lb : lb >> 4) & 15u) | (((hb >> (2 * k)) & 3u) << 4));
        v[l] = (l < 16 ? ds0 : ds1) * (float)(q - 32);
    }
}

__device__ __forceinline__ int q4_block_dot(u32x4 c, const int* xq) {
    // two independent accumulators (low and high nibbles): integer sums, so the split changes nothing but the
    // dependency depth
    int s = 0, u = 0;
    s = __builtin_amdgcn_sdot4((int)(c.x & 0x0F0F0F0Fu), xq[0], s, false);
    u = __builtin_amdgcn_sdot4((int)((c.x >> 4) & 0x0F0F0F0Fu), xq[4], u, false);
    s = __builtin_amdgcn_sdot4((int)(c.y & 0x0F0F0F0Fu), xq[1], s, false);
    u = __builtin_amdgcn_sdot4((int)((c.y >> 4) & 0x0F0F0F0Fu), xq[5], u, false);
    s = __builtin_amdgcn_sdot4((int)(c.z & 0x0F0F0F0Fu), xq[2], s, false);
    u = __builtin_amdgcn_sdot4((int)((c.z >> 4) & 0x0F0F0F0Fu), xq[6], u, false);
    s = __builtin_amdgcn_sdot4((int)(c.w & 0x0F0F0F0Fu), xq[3], s, false);
    u = __builtin_amdgcn_sdot4((int)((c.w >> 4) & 0x0F0F0F0Fu), xq[7], u, false);
    return s + u;
}

// Cut 32 floats to int8 (imi/core/vec.h:47-75): d = amax / 127, id = d ? 1/d : 0, q = round(x * id), returning d
// and the sum of q. half_away selects roundf (imi/kernels/q4x8.cpp:45) instead of round-to-nearest-even.
__device__ __forceinline__ float cut32(const float* v, int* q8, int* sum, bool half_away) {
    float amax = 0.0f;
#pragma unroll
    for (int i = 0; i < 32; i++) amax = fmaxf(amax, fabsf(v[i]));
    const float d = amax / 127.0f;
    const float id = d != 0.0f ? 1.0f / d : 0.0f;
    int s = 0;
#pragma unroll
    for (int w = 0; w < 8; w++) {
        unsigned packed = 0;
#pragma unroll
        for (int b = 0; b < 4; b++) {
            const float t = v[4 * w + b] * id;
            const int c = (int)(half_away ? roundf(t) : rintf(t));
            s += c;
            packed |= ((unsigned)c & 0xFFu) << (8 * b);
        }
        q8[w] = (int)packed;
    }
    *sum = s;
    return d;
}

// e^x, bit for bit glibc's expf (the libm imi runs on). Method: ARM optimized-routines expf (published, used by
// glibc since 2.27): x * 32/ln2 = k + r, 2^(k/32) from a 32-entry table of 2^(i/32) (derived here from the
// mathematics: each entry is 2^(i/32) rounded to double, minus i << 47), times a degree-3 polynomial in r, in
// double with the fused multiply-adds of glibc's FMA build. Exhaustively equal to glibc's expf on all 2^32 inputs.
__constant__ static const uint64_t kExp2Tab[32] = {
    0x3ff0000000000000ull, 0x3fefd9b0d3158574ull, 0x3fefb5586cf9890full, 0x3fef9301d0125b51ull,
    0x3fef72b83c7d517bull, 0x3fef54873168b9aaull, 0x3fef387a6e756238ull, 0x3fef1e9df51fdee1ull,
    0x3fef06fe0a31b715ull, 0x3feef1a7373aa9cbull, 0x3feedea64c123422ull, 0x3feece086061892dull,
    0x3feebfdad5362a27ull, 0x3feeb42b569d4f82ull, 0x3feeab07dd485429ull, 0x3feea47eb03a5585ull,
    0x3feea09e667f3bcdull, 0x3fee9f75e8ec5f74ull, 0x3feea11473eb0187ull, 0x3feea589994cce13ull,
    0x3feeace5422aa0dbull, 0x3feeb737b0cdc5e5ull, 0x3feec49182a3f090ull, 0x3feed503b23e255dull,
    0x3feee89f995ad3adull, 0x3feeff76f2fb5e47ull, 0x3fef199bdd85529cull, 0x3fef3720dcef9069ull,
    0x3fef5818dcfba487ull, 0x3fef7c97337b9b5full, 0x3fefa4afa2a490daull, 0x3fefd0765b6e4540ull};
// tab: the 32-entry table (kExp2Tab, or a copy of it in LDS, which a kernel fills once so that the lookup is not a
// memory round trip)
template <class TabPtr>
__device__ __forceinline__ float expf_glibc_t(float x, TabPtr tab) {
    const uint32_t ux = __float_as_uint(x);
    const uint32_t abstop = (ux >> 20) & 0x7ffu;
    const double inv_ln2_32 = 0x1.71547652b82fep+0 * 32, shift = 0x1.8p+52;
    const double c0 = 0x1.c6af84b912394p-5 / 32 / 32 / 32, c1 = 0x1.ebfce50fac4f3p-3 / 32 / 32, c2 = 0x1.62e42ff0c52d6p-1 / 32;
    const double xd = (double)x;
    double kd = __builtin_fma(inv_ln2_32, xd, shift);
    const uint64_t ki = (uint64_t)__double_as_longlong(kd);
    kd -= shift;
    const double r = __builtin_fma(inv_ln2_32, xd, -kd);
    const uint64_t t = tab[ki & 31] + (ki << 47);
    const double sc = __longlong_as_double((long long)t);
    const double z = __builtin_fma(c0, r, c1);
    const double r2 = r * r;
    double y = __builtin_fma(c2, r, 1.0);
    y = __builtin_fma(z, r2, y);
    // the special cases (|x| >= 88, inf, nan) as selects over the main path's value, the test taken first applied
    // last: no branches, so the evaluations of several values interleave (the main path's table index stays in
    // 0..31 for any input)
    float e = (float)(y * sc);
    e = x < -0x1.9fe368p6f ? 0.0f : e;
    e = x > 0x1.62e42ep6f ? __builtin_inff() : e;
    e = abstop >= 0x7f8u ? x + x : e;               // +inf or nan
    e = ux == 0xff800000u ? 0.0f : e;               // -inf
    return e;
}

__device__ __forceinline__ float expf_glibc(float x) { return expf_glibc_t(x, kExp2Tab); }

__device__ __forceinline__ float silu(float x) { return x / (1.0f + expf_glibc(-x)); }   // imi/core/seoul.cpp:48
template <class TabPtr>
__device__ __forceinline__ float silu_t(float x, TabPtr tab) { return x / (1.0f + expf_glibc_t(-x, tab)); }

// imi_rms_scale (imi/core/vec.h:20-33) in its AVX2 op order, by one whole wave over n floats in LDS
// (n % 32 == 0): partial P (= accumulator P / 8, lane P % 8) is the FMA chain of x[32t + P]^2 over t; then
// v_l = (a0_l + a1_l) + (a2_l + a3_l) and the 8-lane sum ((v0+v4) + (v2+v6)) + ((v1+v5) + (v3+v7));
// returns 1 / sqrtf(s / n + eps) in every lane
template <class Ptr>
__device__ __forceinline__ float rms_scale_wave(Ptr x, int n, float eps) {
    const int lane = threadIdx.x & 63;
    float a = 0.0f;
    if (lane < 32) {   // operands fetched 8 at a time, one batch ahead of the chain that consumes them
        const int nt = n / 32;
        int t = 0;
        if (nt >= 8) {
            float v0[8], v1[8];
#pragma unroll
            for (int q = 0; q < 8; q++) v0[q] = x[32 * q + lane];
            for (; t + 16 <= nt; t += 16) {
#pragma unroll
                for (int q = 0; q < 8; q++) v1[q] = x[32 * (t + 8 + q) + lane];
#pragma unroll
                for (int q = 0; q < 8; q++) a = fmaf(v0[q], v0[q], a);
                if (t + 16 + 8 <= nt) {
#pragma unroll
                    for (int q = 0; q < 8; q++) v0[q] = x[32 * (t + 16 + q) + lane];
                }
#pragma unroll
                for (int q = 0; q < 8; q++) a = fmaf(v1[q], v1[q], a);
            }
            if (t + 8 <= nt) {   // one loaded batch left
#pragma unroll
                for (int q = 0; q < 8; q++) a = fmaf(v0[q], v0[q], a);
                t += 8;
            }
        }
        for (; t < nt; t++) a = fmaf(x[32 * t + lane], x[32 * t + lane], a);
    }
    const float a1 = __shfl(a, (lane + 8) & 63), a2 = __shfl(a, (lane + 16) & 63), a3 = __shfl(a, (lane + 24) & 63);
    const float v = (a + a1) + (a2 + a3);            // lanes 0..7
    const float r = v + __shfl(v, (lane + 4) & 63);  // lanes 0..3: v_l + v_{l+4}
    const float q = r + __shfl(r, (lane + 2) & 63);  // lane 0: (r0 + r2), lane 1: (r1 + r3)
    const float s = __shfl(q, 0) + __shfl(q, 1);
    return 1.0f / sqrtf(s / (float)n + eps);
}

// rms_scale_wave's values (the same chains and combine) for a row of exactly 32 NT values in global memory: every
// operand is requested before the chains start (one memory round trip; fetched a batch ahead of the chains, as from
// LDS, each batch of a row from memory was a round trip of its own)
template <int NT, class Ptr>
__device__ __forceinline__ float rms_scale_wave_g(Ptr x, float eps) {
    constexpr int n = 32 * NT;
    const int lane = threadIdx.x & 63;
    float a = 0.0f;
    if (lane < 32) {
        float v[NT];
#pragma unroll
        for (int t = 0; t < NT; t++) v[t] = x[32 * t + lane];
#pragma unroll
        for (int t = 0; t < NT; t++) a = fmaf(v[t], v[t], a);
    }
    const float a1 = __shfl(a, (lane + 8) & 63), a2 = __shfl(a, (lane + 16) & 63), a3 = __shfl(a, (lane + 24) & 63);
    const float v = (a + a1) + (a2 + a3);            // lanes 0..7
    const float r = v + __shfl(v, (lane + 4) & 63);  // lanes 0..3: v_l + v_{l+4}
    const float q = r + __shfl(r, (lane + 2) & 63);  // lane 0: (r0 + r2), lane 1: (r1 + r3)
    const float s = __shfl(q, 0) + __shfl(q, 1);
    return 1.0f / sqrtf(s / (float)n + eps);
}

// q or k of one head: norm (imi's order) times its weight, then the NEOX rope with the host's cos/sin row of this
// position (imi/core/seoul.cpp:19-28). One wave; lane holds dimensions lane + 64 c (c < DPL), so at D 128 a rope pair
// (i, i + 64) sits in one lane and at D <= 64 the partner comes by a shuffle. stg: D floats of staging.
template <int DPL, class Ptr>
__device__ __forceinline__ void norm_rope_vals(const float (&x)[DPL], const float (&w)[DPL], Ptr stg, const float2 (&cz)[DPL],
                                               int D, float eps, float* r) {
    const int lane = threadIdx.x & 63, half = D / 2;
    float n[DPL];
#pragma unroll
    for (int c = 0; c < DPL; c++)
        if (lane + 64 * c < D) stg[lane + 64 * c] = x[c];
    __builtin_amdgcn_wave_barrier();
    const float s = rms_scale_wave(stg, D, eps);
#pragma unroll
    for (int c = 0; c < DPL; c++) n[c] = lane + 64 * c < D ? x[c] * s * w[c] : 0.0f;
    const float sh = __shfl(n[0], lane < half ? lane + half : lane - half);
#pragma unroll
    for (int c = 0; c < DPL; c++) {
        const int e = lane + 64 * c;
        const float other = DPL == 2 ? n[c ^ 1] : sh;
        r[c] = e < half ? fmaf(n[c], cz[c].x, -(other * cz[c].y)) : fmaf(other, cz[c].y, n[c] * cz[c].x);
    }
    __builtin_amdgcn_wave_barrier();
}
// the operands of one head row: its values (0 past D), the norm weights, the rotation entries of this lane's dimensions
template <int DPL>
__device__ __forceinline__ void norm_rope_load(const float* src, const float* w, const float2* cs, int D, float (&x)[DPL],
                                               float (&wv)[DPL], float2 (&cz)[DPL]) {
    const int lane = threadIdx.x & 63, half = D / 2;
#pragma unroll
    for (int c = 0; c < DPL; c++) {
        const int e = lane + 64 * c;
        x[c] = e < D ? src[e] : 0.0f;
        wv[c] = e < D ? w[e] : 0.0f;
        cz[c] = cs[e < half ? e : (e < D ? e - half : 0)];
    }
}
template <int DPL, class Ptr>
__device__ __forceinline__ void head_norm_rope(const float* src, const float* w, Ptr stg, const float2* cs, int D, float eps, float* r) {
    float x[DPL], wv[DPL];
    float2 cz[DPL];
    norm_rope_load<DPL>(src, w, cs, D, x, wv, cz);
    norm_rope_vals<DPL>(x, wv, stg, cz, D, eps, r);
}

// cross-lane moves on the VALU (DPP), no LDS round trip: lane i gets lane i ^ 1, i ^ 2 (within a quad), 7 - i
// (within 8 lanes), 15 - i (within 16 lanes)
template <int CTRL>
__device__ __forceinline__ float dppf(float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xF, 0xF, true));
}
template <int CTRL>
__device__ __forceinline__ int dppi(int v) { return __builtin_amdgcn_update_dpp(0, v, CTRL, 0xF, 0xF, true); }
constexpr int DPP_XOR1 = 0xB1, DPP_XOR2 = 0x4E, DPP_MIRROR8 = 0x141, DPP_MIRROR16 = 0x140;
template <int CTRL>
__device__ __forceinline__ double dppd(double v) {
    const long long b = __double_as_longlong(v);
    const int lo = dppi<CTRL>((int)b), hi = dppi<CTRL>((int)(b >> 32));
    return __longlong_as_double(((long long)hi << 32) | (unsigned)lo);
}
__device__ __forceinline__ float readlane_f(float v, int l) {
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), l));
}
__device__ __forceinline__ double readlane_d(double v, int l) {
    const long long b = __double_as_longlong(v);
    const unsigned lo = (unsigned)__builtin_amdgcn_readlane((int)b, l), hi = (unsigned)__builtin_amdgcn_readlane((int)(b >> 32), l);
    return __longlong_as_double((long long)(((unsigned long long)hi << 32) | lo));
}
// the wave's maximum in every lane (the wave fully active): four DPP levels leave each 16-lane row's maximum in all
// of its lanes, then the four rows' values are combined (no LDS round trip, unlike a shuffle tree)
__device__ __forceinline__ float wave_max_dpp(float v) {
    v = fmaxf(v, dppf<DPP_XOR1>(v));
    v = fmaxf(v, dppf<DPP_XOR2>(v));
    v = fmaxf(v, dppf<DPP_MIRROR8>(v));
    v = fmaxf(v, dppf<DPP_MIRROR16>(v));
    return fmaxf(fmaxf(readlane_f(v, 0), readlane_f(v, 16)), fmaxf(readlane_f(v, 32), readlane_f(v, 48)));
}

// imi_rms_scale (imi/core/vec.h:20-33) of n = 128 NQ values held transposed (value i at row i % 32, column i / 32,
// rows LD floats apart; 16-byte aligned rows), by one wave. imi's order: 32 FMA chains, chain P
// over the squares of values P, P + 32, P + 64, ...; then v_P = (a_P + a_{P+8}) + (a_{P+16} + a_{P+24}) for P < 8 and
// ((v0 + v4) + (v2 + v6)) + ((v1 + v5) + (v3 + v7)). Lane L < 32 runs chain P(L) = 8 b0 + 16 b1 + 4 b2 + 2 b3 + b4
// (b_k = bit k of L), so the tree's levels pair lanes L ^ 1, ^ 2, then 8-lane and 16-lane mirrors, then 0 and 16:
// each level is one DPP add (fp addition is commutative, so the pair order does not matter, only the tree).
// Every lane gets 1 / sqrtf(s / n + eps).
template <class P> struct quad_of;   // float pointer -> f32x4 pointer in the same address space
template <> struct quad_of<const float*> { typedef const f32x4* type; };
template <> struct quad_of<const float __attribute__((address_space(3)))*> {
    typedef const f32x4 __attribute__((address_space(3)))* type;
};

template <int NQ, int LD, class Ptr>
__device__ __forceinline__ float rms_scale_xt(Ptr xt, float eps) {
    const int lane = threadIdx.x & 63;
    const int row = 8 * (lane & 1) + 16 * ((lane >> 1) & 1) + 4 * ((lane >> 2) & 1) + 2 * ((lane >> 3) & 1) + ((lane >> 4) & 1);
    const auto r = (typename quad_of<Ptr>::type)(xt + row * LD);
    constexpr int B = NQ < 8 ? NQ : 8;   // quads per batch; the next batch is read while this one runs
    float a = 0.0f;
    f32x4 cur[B], nxt[B];
#pragma unroll
    for (int k = 0; k < B; k++) cur[k] = r[k];
#pragma unroll
    for (int q = 0; q < NQ; q += B) {
        if (q + B < NQ) {
#pragma unroll
            for (int k = 0; k < B; k++) nxt[k] = r[q + B + k];
        }
#pragma unroll
        for (int k = 0; k < B; k++) {
            a = fmaf(cur[k].x, cur[k].x, a);
            a = fmaf(cur[k].y, cur[k].y, a);
            a = fmaf(cur[k].z, cur[k].z, a);
            a = fmaf(cur[k].w, cur[k].w, a);
        }
        if (q + B < NQ) {
#pragma unroll
            for (int k = 0; k < B; k++) cur[k] = nxt[k];
        }
    }
    float x = a;   // lanes 32..63 ran the same chains; only lanes 0..31 are read below
    x = x + dppf<DPP_XOR1>(x);
    x = x + dppf<DPP_XOR2>(x);
    x = x + dppf<DPP_MIRROR8>(x);
    x = x + dppf<DPP_MIRROR16>(x);
    const float s = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(x), 0)) +
                    __int_as_float(__builtin_amdgcn_readlane(__float_as_int(x), 16));
    return 1.0f / sqrtf(s / (float)(128 * NQ) + eps);
}

// A pointer a kernel reads from memory (the step parameter block: K/V caches, conv memory, output ids) is generic to
// the compiler, so every access through it becomes a flat instruction, and a flat load counts against the LDS wait
// counter as well as the vector-memory one: each wait for an LDS result then also waits for that load to come back
// from memory. The pointers held there are all device memory; this says so (the cast to the global address space
// lets the compiler use global instructions for every access through the result, which keeps the address space in
// its type: a cast back to a generic pointer would be folded away with it).
#define SH_GLOBAL __attribute__((address_space(1)))
template <class T>
__device__ __forceinline__ SH_GLOBAL T* global_ptr(T* p) {
    return (SH_GLOBAL T*)p;
}

// dot_h (imi/core/seoul.cpp:29-39): 8 FMA chains over columns i % 8, then the 8-lane horizontal sum
template <int D>
__device__ __forceinline__ float dot_h8(const float* q, const float* k) {
    float a[8];
#pragma unroll
    for (int l = 0; l < 8; l++) a[l] = 0.0f;
#pragma unroll
    for (int i = 0; i < D; i += 8)
#pragma unroll
        for (int l = 0; l < 8; l++) a[l] = fmaf(q[i + l], k[i + l], a[l]);
    return ((a[0] + a[4]) + (a[2] + a[6])) + ((a[1] + a[5]) + (a[3] + a[7]));
}

// device-scope (sc1) stores/loads for values another block reads in the same kernel (no whole-cache fences)
__device__ __forceinline__ void st_dev(float* p, float v) { __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT); }
__device__ __forceinline__ void st_dev(int* p, int v) { __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT); }

}  // namespace sh
