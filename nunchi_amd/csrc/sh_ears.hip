// Kernels of the ears (imi/core/ears.cpp:198-407) for gfx950. Every fp32 operation is the one the oracle
// restatement of imi's ears performs, in the same order; the exceptions are the C library's erff (GELU) and the
// double log10 of the mel, here the device's routines.
//
// The float tables run on the matrix cores in imi_wg_group12's order (k_etab below).
#include "sh_ears.h"
#include "sh_device.h"

namespace sh {
namespace {

constexpr int ET = 256;

__device__ __forceinline__ float gelu_erf(float x) { return 0.5f * x * (1.0f + erff(x * 0.70710678118654752f)); }

// imi_rms_scale (imi/core/vec.h:20-33) in its AVX2 op order by one half-wave over one row of n floats (n % 32 == 0):
// lane P of the half runs the fma chain of x[32t + P]^2 over t (all loads issued first, 8 at a time), then
// v_l = (a_l + a_{l+8}) + (a_{l+16} + a_{l+24}) and ((v0+v4) + (v2+v6)) + ((v1+v5) + (v3+v7)); every lane of the
// half gets 1 / sqrtf(s / n + eps)
__device__ __forceinline__ float rms_scale_half(const float* x, int n, float eps) {
    const int lane = threadIdx.x & 63, hl = lane & 31, base = lane & 32;
    const int nt = n / 32;
    float a = 0.0f;
    int t = 0;
    for (; t + 8 <= nt; t += 8) {
        float v[8];
#pragma unroll
        for (int q = 0; q < 8; q++) v[q] = x[32 * (t + q) + hl];
#pragma unroll
        for (int q = 0; q < 8; q++) a = fmaf(v[q], v[q], a);
    }
    for (; t < nt; t++) a = fmaf(x[32 * t + hl], x[32 * t + hl], a);
    auto at = [&](float v, int l) { return __shfl(v, base + (l & 31)); };
    const float v = (a + at(a, hl + 8)) + (at(a, hl + 16) + at(a, hl + 24));   // lanes 0..7 of the half
    const float r = v + at(v, hl + 4);
    const float q = r + at(r, hl + 2);
    const float s = at(q, 0) + at(q, 1);
    return 1.0f / sqrtf(s / (float)n + eps);
}


// 8 columns of one row, raw: F16 bits (one 16-byte load) or F32 (two)
template <bool F32W> struct wraw;
template <> struct wraw<false> { uint4 a; };
template <> struct wraw<true> { float4 a, b; };

template <bool F32W>
__device__ __forceinline__ wraw<F32W> wload(const void* w, size_t at) {
    wraw<F32W> r;
    if constexpr (F32W) {
        const float4* p = static_cast<const float4*>(w) + at * 2;
        r.a = p[0];
        r.b = p[1];
    } else {
        r.a = static_cast<const uint4*>(w)[at];
    }
    return r;
}
template <bool F32W>
__device__ __forceinline__ void wconv(const wraw<F32W>& r, float (&o)[8]) {
    if constexpr (F32W) {
        o[0] = r.a.x; o[1] = r.a.y; o[2] = r.a.z; o[3] = r.a.w; o[4] = r.b.x; o[5] = r.b.y; o[6] = r.b.z; o[7] = r.b.w;
    } else {
        const unsigned v[4] = {r.a.x, r.a.y, r.a.z, r.a.w};
#pragma unroll
        for (int i = 0; i < 4; i++) {
            o[2 * i] = h2f((uint16_t)(v[i] & 0xffffu));
            o[2 * i + 1] = h2f((uint16_t)(v[i] >> 16));
        }
    }
}

// The float tables on the matrix cores, in imi_wg_group12's order (imi/core/tables.cpp:522-556): one chain
// acc = fma(w, x, acc) per row and position over the columns in order. v_mfma_f32_4x4x1_16b_f32 forms
// d[l][i] = fma(a[4 (l / 4) + i], b[l], c[l][i]) with one rounding, bit for bit the VALU's fmaf (measured over 10^6
// random cases with denormals, signed zeros and fused cancellation), so one instruction per column advances 16 blocks
// of 4 rows x 4 positions of those chains by one step each, in column order. Lane l supplies its own row's weight (a)
// and the input of position l % 4 (b); it holds rows 4 (l / 4) .. + 3 of position l % 4. A workgroup is 64 rows by
// 4 waves x NMF position quads (NMF instructions per column and wave, one weight conversion); a wave keeps DW weight
// loads in flight and stages its inputs position-major in LDS 128 columns at a time (one chunk ahead), 8 columns read
// per 16-byte pair (a broadcast of the same word to every lane would cost the LDS its full return bandwidth). Every
// global load is unconditional (indices clamped into the buffers; no product reads a column past the table, whose
// width is a multiple of 8), so the compiler's wait counts stay exact.
template <int EPI, bool F32W, int NMF>
__global__ __launch_bounds__(ET) void k_etab(etab_args a) {
    typedef float v4f __attribute__((ext_vector_type(4)));
    constexpr int KC = 128, KCP = KC + 4, DW = 8, NP = 4 * NMF;
    __shared__ __align__(16) float xs[ET / 64][2][NP][KCP];
    constexpr bool EXPE = EPI == EE_GLU || EPI == EE_SILU;   // epilogues that take e^x
    __shared__ uint64_t eE[ET / 64][EXPE ? 32 : 1];         // expf's table, a copy per wave (no memory round trip)
    const int lane = threadIdx.x & 63, wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), q = lane & 3;
    const uint64_t et = EXPE ? kExp2Tab[lane & 31] : 0;      // (requested first: its wait needs nothing later)
    const int r = blockIdx.x * 64 + lane, p0 = (blockIdx.y * 4 + wv) * NP;
    const int rp = a.W.rows_pad, K = a.W.cols, nk8 = K >> 3, nch = (K + KC - 1) / KC;
    const size_t ldx = (size_t)a.ldx;
    const int rr = r < rp ? r : rp - 1;   // lanes past the table read its last row (nothing stored)
    float4 st[KC / 64][NMF];
    wraw<F32W> wq[DW];
#pragma unroll
    for (int i = 0; i < DW; i++) wq[i] = wload<F32W>(a.W.w, (size_t)(i < nk8 ? i : nk8 - 1) * rp + rr);
    v4f acc[NMF];
#pragma unroll
    for (int m = 0; m < NMF; m++) acc[m] = v4f{0.0f, 0.0f, 0.0f, 0.0f};
    for (int c = -1; c < nch; c++) {
        // chunk c + 1's inputs are requested (clamped to the last chunk), chunk c runs from LDS, then c + 1 is stored
        {
            const int cn = c + 1 < nch ? c + 1 : nch - 1;
#pragma unroll
            for (int i = 0; i < KC / 64; i++) {
                const int k = min(cn * KC + lane + 64 * i, K - 1);
#pragma unroll
                for (int m = 0; m < NMF; m++) {
                    const int pm = min(p0 + 4 * m, a.ldx - 4);
                    st[i][m] = *reinterpret_cast<const float4*>(a.x + (size_t)k * ldx + pm);
                }
            }
        }
        if (c >= 0) {
            const float* xc = &xs[wv][c & 1][0][0];
            const int kb0 = c * (KC / 8);
#pragma unroll
            for (int u = 0; u < KC / 8; u++) {   // the ring slot u % DW is static (KC / 8 is a multiple of DW)
                const int kb = kb0 + u, kn = kb + DW < nk8 ? kb + DW : nk8 - 1;
                float w[8];
                wconv<F32W>(wq[u % DW], w);
                wq[u % DW] = wload<F32W>(a.W.w, (size_t)kn * rp + rr);
                if (kb < nk8) {
                    float xv[NMF][8];
#pragma unroll
                    for (int m = 0; m < NMF; m++) {
                        const float* xp = xc + (4 * m + q) * KCP + 8 * u;
                        const float4 x0 = *reinterpret_cast<const float4*>(xp), x1 = *reinterpret_cast<const float4*>(xp + 4);
                        xv[m][0] = x0.x; xv[m][1] = x0.y; xv[m][2] = x0.z; xv[m][3] = x0.w;
                        xv[m][4] = x1.x; xv[m][5] = x1.y; xv[m][6] = x1.z; xv[m][7] = x1.w;
                    }
#pragma unroll
                    for (int j = 0; j < 8; j++)
#pragma unroll
                        for (int m = 0; m < NMF; m++) acc[m] = __builtin_amdgcn_mfma_f32_4x4x1f32(w[j], xv[m][j], acc[m], 0, 0, 0);
                }
            }
        }
        __builtin_amdgcn_wave_barrier();
        if (c + 1 < nch) {
#pragma unroll
            for (int i = 0; i < KC / 64; i++)
#pragma unroll
                for (int m = 0; m < NMF; m++) {
                    float* xw = &xs[wv][(c + 1) & 1][4 * m][lane + 64 * i];
                    xw[0] = st[i][m].x;
                    xw[KCP] = st[i][m].y;
                    xw[2 * KCP] = st[i][m].z;
                    xw[3 * KCP] = st[i][m].w;
                }
        }
        __builtin_amdgcn_wave_barrier();
    }
    // lane l holds rows rb .. rb + 3 of position p0 + 4 m + l % 4 (rb = the workgroup's first row + 4 (l / 4))
    const int rb = blockIdx.x * 64 + 4 * (lane >> 2);
    if (EXPE && lane < 32) eE[wv][EXPE ? lane : 0] = et;
    __builtin_amdgcn_wave_barrier();
    const uint64_t* etab = eE[wv];
    const bool xt = a.xt_out;
    const int pend = xt ? min(a.ldx, a.ldo) : a.P;   // the feature-major output also fills the padded positions
    auto put = [&](int row, int p, float v) {
        float* d = xt ? a.out + (size_t)row * a.ldo + p : a.out + (size_t)p * a.ldo + row;
        *d = EPI == EE_ADD ? *d + v : v;
    };
#pragma unroll
    for (int m = 0; m < NMF; m++) {
        const int p = p0 + 4 * m + q;
        if constexpr (EPI == EE_GLU) {   // rows 0-7 of each 16 are gates, 8-15 the matching ups (lanes + 8)
            v4f up;
#pragma unroll
            for (int i = 0; i < 4; i++) up[i] = __shfl_xor(acc[m][i], 8);
            if ((lane & 8) == 0 && p < pend) {
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    const int row = rb + i, ro = (row >> 4) * 8 + (row & 7);
                    if (ro < a.W.rows / 2) put(ro, p, silu_t(acc[m][i], etab) * up[i]);
                }
            }
        } else if constexpr (EPI == EE_POWER) {   // rows (2j, 2j + 1) = (re, im) of bin j
            if (p < pend) {
#pragma unroll
                for (int h = 0; h < 2; h++) {
                    const int ro = (rb >> 1) + h;
                    if (ro < a.W.rows / 2) put(ro, p, fmaf(acc[m][2 * h], acc[m][2 * h], acc[m][2 * h + 1] * acc[m][2 * h + 1]));
                }
            }
        } else if (p < pend) {
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const int row = rb + i;
                if (row >= a.W.rows) break;
                const float v = acc[m][i] + (a.bias ? a.bias[row] : 0.0f);
                put(row, p, EPI == EE_SILU ? silu_t(v, etab) : EPI == EE_GELU ? gelu_erf(v) : v);
            }
        }
    }
}

__global__ __launch_bounds__(ET) void k_eframes(const float* pcm, int n, const float* hann, int n_fft, int hop,
                                                int n_fr, float* fx, int ldf) {
    const int fr = blockIdx.x * ET + threadIdx.x, k = blockIdx.y;
    if (fr >= ldf) return;
    const long i = (long)fr * hop + k;
    fx[(size_t)k * ldf + fr] = fr < n_fr && i < n ? hann[k] * pcm[i] : 0.0f;
}

// imi sums all n_bin terms in bin order; a term with a zero filter weight is fma(0, pw, s) = s exactly (pw is a sum of
// two squares, finite and >= 0), so each mel only runs over its filter's nonzero bins [lo, hi), in order
__global__ __launch_bounds__(ET) void k_emel(const float* pw, int ldp, const float* fb, const int2* span, int n_bin,
                                             int n_mel, int n_fr, float* mel) {
    const int fr = blockIdx.x * ET + threadIdx.x, m = blockIdx.y;
    if (fr >= n_fr) return;
    const float* w = fb + (size_t)m * n_bin;
    const int2 sp = span[m];
    double s = 0.0;
    for (int b = sp.x; b < sp.y; b++) s = fma((double)w[b], (double)pw[(size_t)b * ldp + fr], s);
    mel[(size_t)fr * n_mel + m] = (float)((log10(s < 1e-12 ? 1e-12 : s) + 4.0) / 4.0);
}

// thread per (t, f) and 8 channels: the 9 taps' inputs are requested first (addresses clamped into the image) and
// shared by the channels; a tap outside the image leaves o as it is (a select, not a multiply by zero, so o keeps its
// bits exactly as imi's skipped tap does)
constexpr int E0_CPT = 8;
__global__ __launch_bounds__(ET) void k_econv0(const float* mel, int n_fr, int n_mel, const float* w9, const float* b,
                                               int C, int T2, int F2, float* a0) {
    const int i = blockIdx.x * ET + threadIdx.x, c0 = blockIdx.y * E0_CPT;
    if (i >= T2 * F2) return;
    const int t = i / F2, f = i - t * F2;
    float v[9];
    bool ok[9];
#pragma unroll
    for (int j = 0; j < 9; j++) {
        const int ti = 2 * t + j % 3 - 1, fi = 2 * f + j / 3 - 1;   // j = kh * 3 + kw: kw along time, kh along freq
        ok[j] = ti >= 0 && ti < n_fr && fi >= 0 && fi < n_mel;
        const int tc = ti < 0 ? 0 : ti >= n_fr ? n_fr - 1 : ti, fc = fi < 0 ? 0 : fi >= n_mel ? n_mel - 1 : fi;
        v[j] = mel[(size_t)tc * n_mel + fc];
    }
#pragma unroll
    for (int cc = 0; cc < E0_CPT; cc++) {
        const int c = c0 + cc;
        if (c >= C) break;
        float o = b[c];
#pragma unroll
        for (int j = 0; j < 9; j++) {
            const float u = fmaf(v[j], w9[(size_t)j * C + c], o);
            o = ok[j] ? u : o;
        }
        a0[(size_t)c * T2 * F2 + i] = silu(o);
    }
}

__global__ __launch_bounds__(ET) void k_edw(const float* in, int Ti, int Fi, int ldi, const float* w9, const float* b,
                                            int C, int To, int Fo, float* out, int ldo) {
    const int i = blockIdx.x * ET + threadIdx.x, c = blockIdx.y;
    if (i >= To * Fo) return;
    const int t = i / Fo, f = i - t * Fo;
    const float* src = in + (size_t)c * ldi;
    float v[9];
    bool ok[9];
#pragma unroll
    for (int j = 0; j < 9; j++) {
        const int ti = 2 * t + j % 3 - 1, fi = 2 * f + j / 3 - 1;
        ok[j] = ti >= 0 && ti < Ti && fi >= 0 && fi < Fi;
        const int tc = ti < 0 ? 0 : ti >= Ti ? Ti - 1 : ti, fc = fi < 0 ? 0 : fi >= Fi ? Fi - 1 : fi;
        v[j] = src[(size_t)tc * Fi + fc];
    }
    float o = b[c];
#pragma unroll
    for (int j = 0; j < 9; j++) {
        const float u = fmaf(v[j], w9[(size_t)j * C + c], o);
        o = ok[j] ? u : o;
    }
    out[(size_t)c * ldo + (size_t)t * Fo + f] = o;
}

__global__ __launch_bounds__(ET) void k_eflat(const float* a, int lda, int F8, int P, float* xf, int ldf) {
    const int p = blockIdx.x * ET + threadIdx.x, k = blockIdx.y;
    if (p >= ldf) return;
    const int c = k / F8, f = k - c * F8;
    xf[(size_t)k * ldf + p] = p < P ? a[(size_t)c * lda + (size_t)p * F8 + f] : 0.0f;
}

// a workgroup is 16 positions x 64 features: each wave forms 4 positions' scales in imi's order (every workgroup of a
// position forms the same scale), then h is written feature-major, 16 positions (64 bytes) per feature row
__global__ __launch_bounds__(ET) void k_enorm(const float* x, const float* w, int E, int P, int ldh, float eps, float* h) {
    __shared__ float sc[16];
    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6, p0 = blockIdx.x * 16, e0 = blockIdx.y * 64;
    for (int q = 0; q < 2; q++) {   // half-wave hf forms position p0 + 4 wv + 2 q + hf
        const int hf = lane >> 5, pq = wv * 4 + 2 * q + hf, p = p0 + pq;
        const float s = rms_scale_half(x + (size_t)(p < P ? p : 0) * E, E, eps);
        if ((lane & 31) == 0) sc[pq] = p < P ? s : 0.0f;
    }
    __syncthreads();
    const int pl = threadIdx.x & 15, p = p0 + pl;
    const float s = sc[pl];
    for (int e = e0 + (threadIdx.x >> 4); e < e0 + 64 && e < E; e += ET / 16)
        h[(size_t)e * ldh + p] = p < P ? x[(size_t)p * E + e] * s * w[e] : 0.0f;
}

__global__ __launch_bounds__(ET) void k_econv(const float* big, int ld, const float* w, int E, int d_conv, int P,
                                              float* act, int lda) {
    const int e = blockIdx.x * ET + threadIdx.x, p = blockIdx.y;
    if (e >= E) return;
    if (p >= P) { act[(size_t)e * lda + p] = 0.0f; return; }
    float co = 0.0f;
    for (int k = 0; k < d_conv; k++) {
        const int t = p - (d_conv - 1) + k;
        if (t < 0) continue;
        const float* rw = big + (size_t)t * ld;
        co = fmaf(w[(size_t)k * E + e], rw[e] * rw[2 * E + e], co);
    }
    act[(size_t)e * lda + p] = big[(size_t)p * ld + E + e] * co;
}

// one wave per (position, head slot): the n_head query heads, then the n_kv key heads
template <int DPL>
__global__ __launch_bounds__(ET) void k_eqk(float* big, int ld, int n_head, int n_kv, int D, const float* q_norm,
                                            const float* k_norm, const float2* cs, int P, float eps) {
    __shared__ float stg[ET / 64][EA_MAX_D];
    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6, ns = n_head + n_kv;
    const int u = blockIdx.x * (ET / 64) + wv;
    if (u >= P * ns) return;
    const int p = u / ns, sl = u - p * ns;
    float* v = big + (size_t)p * ld + (sl < n_head ? sl * D : n_head * D + (sl - n_head) * D);
    float r[DPL];
    head_norm_rope<DPL>(v, sl < n_head ? q_norm : k_norm, stg[wv], cs + (size_t)p * (D / 2), D, eps, r);
#pragma unroll
    for (int c = 0; c < DPL; c++)
        if (lane + 64 * c < D) v[lane + 64 * c] = r[c];
}

// one wave per (position, query head): lane t < nk scores key s0 + t (fma chain over the dimensions), the exponentials
// are summed in key order by lane 0, lane i runs dimension i's chain o = fma(e_t, v_t, o) over the keys
__global__ __launch_bounds__(ET) void k_eattn(const float* big, int ld, int n_head, int n_kv, int D, int window, int P,
                                              float* act, int lda) {
    __shared__ float qs[ET / 64][EA_MAX_D];
    __shared__ float es[ET / 64][EA_MAX_WIN];
    __shared__ float sums[ET / 64];
    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
    const int u = blockIdx.x * (ET / 64) + wv;
    if (u >= P * n_head) return;
    const int p = u / n_head, hh = u - p * n_head, kv = hh / (n_head / n_kv);
    const int Hq = n_head * D, Hk = n_kv * D;
    const int s0 = p - window + 1 > 0 ? p - window + 1 : 0, nk = p - s0 + 1;
    for (int i = lane; i < D; i += 64) qs[wv][i] = big[(size_t)p * ld + hh * D + i];
    __builtin_amdgcn_wave_barrier();
    const float scale = 1.0f / sqrtf((float)D);
    float sc = -__builtin_inff();
    if (lane < nk) {
        const float* k = big + (size_t)(s0 + lane) * ld + Hq + kv * D;
        float s = 0.0f;
        for (int i = 0; i < D; i++) s = fmaf(qs[wv][i], k[i], s);
        sc = s * scale;
    }
    float mx = sc;
    for (int o = 32; o > 0; o >>= 1) {
        const float t = __shfl_xor(mx, o);
        mx = mx < t ? t : mx;
    }
    if (lane < nk) es[wv][lane] = expf_glibc(sc - mx);
    __builtin_amdgcn_wave_barrier();
    if (lane == 0) {
        float sum = 0.0f;
        for (int t = 0; t < nk; t++) sum += es[wv][t];
        sums[wv] = sum;
    }
    __builtin_amdgcn_wave_barrier();
    const float sum = sums[wv];
    for (int i = lane; i < D; i += 64) {
        float o = 0.0f;
        for (int t = 0; t < nk; t++) o = fmaf(es[wv][t], big[(size_t)(s0 + t) * ld + Hq + Hk + kv * D + i], o);
        act[(size_t)(hh * D + i) * lda + p] = o / sum;
    }
}

// one wave per position: h = x * rms(x) * post_ln into LDS; lane 0 forms the double mean and variance in order;
// then fma((float)(h - mu) * inv, ln_w, ln_b)
__global__ __launch_bounds__(ET) void k_efinal(const float* x, const float* post_ln, const float* ln_w,
                                               const float* ln_b, int E, int P, float eps, float* h, int ldh) {
    extern __shared__ float hs_all[];
    __shared__ double st[ET / 64][2];
    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6, p = blockIdx.x * (ET / 64) + wv;
    if (p >= ldh) return;
    if (p >= P) {
        for (int e = lane; e < E; e += 64) h[(size_t)e * ldh + p] = 0.0f;
        return;
    }
    float* hs = hs_all + (size_t)wv * E;
    const float* xp = x + (size_t)p * E;
    const float s = E == 768 ? rms_scale_wave_g<24>(xp, eps) : rms_scale_wave(xp, E, eps);
    for (int e = lane; e < E; e += 64) hs[e] = xp[e] * s * post_ln[e];
    __builtin_amdgcn_wave_barrier();
    if (lane == 0) {
        double mu = 0.0, var = 0.0;
        for (int k = 0; k < E; k++) mu += (double)hs[k];
        mu /= E;
        for (int k = 0; k < E; k++) {
            const double d = (double)hs[k] - mu;
            var = fma(d, d, var);
        }
        st[wv][0] = mu;
        st[wv][1] = (double)(float)(1.0 / sqrt(var / E + 1e-5));
    }
    __builtin_amdgcn_wave_barrier();
    const double mu = st[wv][0];
    const float inv = (float)st[wv][1];
    for (int e = lane; e < E; e += 64) h[(size_t)e * ldh + p] = fmaf((float)((double)hs[e] - mu) * inv, ln_w[e], ln_b[e]);
}

inline unsigned blocks(long n) { return (unsigned)((n + ET - 1) / ET); }

}  // namespace

hipError_t launch_etab(int epi, const etab_args& a, hipStream_t s) {
    if (a.W.cols % 8 || a.W.rows_pad % 8 || a.ldx % 16 || (a.xt_out && a.ldo % 4) ||
        (epi == EE_GLU && a.W.rows_pad % 16))
        return hipErrorInvalidValue;
    const unsigned gx = (unsigned)((a.W.rows_pad + 63) / 64);
    // position quads per wave: the most that keeps enough waves in flight (the chains are as long as the table is wide)
    const auto waves = [&](int nmf) { return 4L * gx * ((a.ldx + 16 * nmf - 1) / (16 * nmf)); };
    const int nmf = waves(4) >= 2048 ? 4 : waves(2) >= 2048 ? 2 : 1;
    const dim3 grid(gx, (unsigned)((a.ldx + 16 * nmf - 1) / (16 * nmf)));
#define SH_ETAB(E)                                                                                        \
    case E:                                                                                               \
        if (a.W.f32) {                                                                                    \
            if (nmf == 4) SH_ETAB_MF(E, true, 4); else if (nmf == 2) SH_ETAB_MF(E, true, 2); else SH_ETAB_MF(E, true, 1); \
        } else {                                                                                          \
            if (nmf == 4) SH_ETAB_MF(E, false, 4); else if (nmf == 2) SH_ETAB_MF(E, false, 2); else SH_ETAB_MF(E, false, 1); \
        }                                                                                                 \
        break;
#define SH_ETAB_MF(E, F, N) hipLaunchKernelGGL((k_etab<E, F, N>), grid, dim3(ET), 0, s, a)
    switch (epi) {
        SH_ETAB(EE_STORE) SH_ETAB(EE_ADD) SH_ETAB(EE_SILU) SH_ETAB(EE_GELU) SH_ETAB(EE_GLU) SH_ETAB(EE_POWER)
        default: return hipErrorInvalidValue;
    }
#undef SH_ETAB
#undef SH_ETAB_MF
    return hipGetLastError();
}

hipError_t launch_eframes(const float* pcm, int n, const float* hann, int n_fft, int hop, int n_fr, float* fx, int ldf,
                          hipStream_t s) {
    hipLaunchKernelGGL(k_eframes, dim3(blocks(ldf), n_fft), dim3(ET), 0, s, pcm, n, hann, n_fft, hop, n_fr, fx, ldf);
    return hipGetLastError();
}
hipError_t launch_emel(const float* pw, int ldp, const float* fb, const int2* span, int n_bin, int n_mel, int n_fr,
                       float* mel, hipStream_t s) {
    hipLaunchKernelGGL(k_emel, dim3(blocks(n_fr), n_mel), dim3(ET), 0, s, pw, ldp, fb, span, n_bin, n_mel, n_fr, mel);
    return hipGetLastError();
}
hipError_t launch_econv0(const float* mel, int n_fr, int n_mel, const float* w9, const float* b, int C, float* a0,
                         hipStream_t s) {
    const int T2 = (n_fr + 1) / 2, F2 = n_mel / 2;
    hipLaunchKernelGGL(k_econv0, dim3(blocks((long)T2 * F2), (C + E0_CPT - 1) / E0_CPT), dim3(ET), 0, s, mel, n_fr, n_mel,
                       w9, b, C, T2, F2, a0);
    return hipGetLastError();
}
hipError_t launch_edw(const float* in, int Ti, int Fi, int ldi, const float* w9, const float* b, int C, float* out,
                      int ldo, hipStream_t s) {
    const int To = (Ti + 1) / 2, Fo = Fi / 2;
    hipLaunchKernelGGL(k_edw, dim3(blocks((long)To * Fo), C), dim3(ET), 0, s, in, Ti, Fi, ldi, w9, b, C, To, Fo, out, ldo);
    return hipGetLastError();
}
hipError_t launch_eflat(const float* a, int lda, int C, int F8, int P, float* xf, int ldf, hipStream_t s) {
    hipLaunchKernelGGL(k_eflat, dim3(blocks(ldf), C * F8), dim3(ET), 0, s, a, lda, F8, P, xf, ldf);
    return hipGetLastError();
}
hipError_t launch_enorm(const float* x, const float* w, int E, int P, float eps, float* h, int ldh, hipStream_t s) {
    if (E % 32) return hipErrorInvalidValue;
    if (ldh % 16) return hipErrorInvalidValue;
    hipLaunchKernelGGL(k_enorm, dim3((unsigned)(ldh / 16), (unsigned)((E + 63) / 64)), dim3(ET), 0, s, x, w, E, P, ldh, eps, h);
    return hipGetLastError();
}
hipError_t launch_econv(const float* big, int ld, const float* w, int E, int d_conv, int P, float* act, int lda,
                        hipStream_t s) {
    hipLaunchKernelGGL(k_econv, dim3(blocks(E), lda), dim3(ET), 0, s, big, ld, w, E, d_conv, P, act, lda);
    return hipGetLastError();
}
hipError_t launch_eqk(float* big, int ld, int n_head, int n_kv, int D, const float* q_norm, const float* k_norm,
                      const float2* cs, int P, float eps, hipStream_t s) {
    if (D % 32 || D > EA_MAX_D) return hipErrorInvalidValue;
    const unsigned g = (unsigned)(((long)P * (n_head + n_kv) + 3) / 4);
    if (D > 64) hipLaunchKernelGGL((k_eqk<2>), dim3(g), dim3(ET), 0, s, big, ld, n_head, n_kv, D, q_norm, k_norm, cs, P, eps);
    else hipLaunchKernelGGL((k_eqk<1>), dim3(g), dim3(ET), 0, s, big, ld, n_head, n_kv, D, q_norm, k_norm, cs, P, eps);
    return hipGetLastError();
}
hipError_t launch_eattn(const float* big, int ld, int n_head, int n_kv, int D, int window, int P, float* act, int lda,
                        hipStream_t s) {
    if (D > EA_MAX_D || window < 1 || window > EA_MAX_WIN) return hipErrorInvalidValue;
    hipLaunchKernelGGL(k_eattn, dim3((unsigned)(((long)P * n_head + 3) / 4)), dim3(ET), 0, s, big, ld, n_head, n_kv, D,
                       window, P, act, lda);
    return hipGetLastError();
}
hipError_t launch_efinal(const float* x, const float* post_ln, const float* ln_w, const float* ln_b, int E, int P,
                         float eps, float* h, int ldh, hipStream_t s) {
    if (E % 32 || E > 4096) return hipErrorInvalidValue;
    hipLaunchKernelGGL(k_efinal, dim3((unsigned)((ldh + 3) / 4)), dim3(ET), (size_t)4 * E * sizeof(float), s, x, post_ln,
                       ln_w, ln_b, E, P, eps, h, ldh);
    return hipGetLastError();
}

}  // namespace sh
