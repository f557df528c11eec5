// Kernels of the codec decoder (imi/core/codec.cpp:121-277) for gfx950: the frame's vector, the conv and attention
// parts of its LFM layers, the post-norm residuals and the inverse STFT. The Q8_0 table products are the voice
// generator's kernels. Every fp32 operation is the one the oracle restatement of imi's codec performs, in the same
// order; the one difference is the cosine and sine of each bin's phase (the device's double-precision routines
// rounded to float, where imi calls the C library's cosf / sinf).
#include "sh_codec.h"
#include "sh_device.h"

namespace sh {
namespace {

constexpr int CX_MAX_E = 512;   // codec width the attention kernel stages (the head gates read the layer input)
constexpr int CX_NT = 256;

// codes -> levels -> s = b[o] + sum_i w[o][i] q[i] as one fma chain from the bias (codec.cpp:147-152)
__global__ __launch_bounds__(CX_NT) void k_cfsq(cfsq_args a) {
    __shared__ float q[CX_NCB * 16];
    const int nq = CX_NCB * a.n_lvl;
    for (int i = threadIdx.x; i < nq; i += CX_NT) {
        const int cb = i / a.n_lvl, l = i - cb * a.n_lvl;
        q[i] = a.lvl[(size_t)a.in->codes[cb] * a.n_lvl + l];
    }
    __syncthreads();
    for (int o = threadIdx.x; o < a.n_q; o += CX_NT) {
        float s = a.b[o];
        const float* w = a.w + (size_t)o * nq;
        for (int i = 0; i < nq; i++) s = fmaf(w[i], q[i], s);
        a.out[o] = s;
    }
}

__global__ __launch_bounds__(CX_NT) void k_crep(crep_args a) {
    const int i = blockIdx.x * CX_NT + threadIdx.x;
    if (i < (CX_P - 1) * a.E) a.x[a.E + i] = a.x[i % a.E];
}

// thread per channel: bx = b * x per position, u = c * sum over taps k of fma(src_k, w_k, u) in tap order, src
// running over [memory (d_conv rows) | bx (P rows)]; then the memory keeps the last d_conv rows of that sequence
__global__ __launch_bounds__(CX_NT) void k_cconv(cconv_args a) {
    const int e = blockIdx.x * CX_NT + threadIdx.x, E = a.E, dc = a.d_conv;
    if (e >= E) return;
    float all[CX_MAX_TAPS - 1 + CX_P], w[CX_MAX_TAPS];
#pragma unroll
    for (int k = 0; k < CX_MAX_TAPS - 1; k++) all[k] = k < dc ? a.mem[(size_t)k * E + e] : 0.0f;
#pragma unroll
    for (int k = 0; k < CX_MAX_TAPS; k++) w[k] = k <= dc ? a.taps[(size_t)k * E + e] : 0.0f;
    // the sequence [memory | bx] with the memory right-aligned at index dc - 1
    float seq[CX_MAX_TAPS - 1 + CX_P];
#pragma unroll
    for (int p = 0; p < CX_P; p++) {
        const float* r = a.big + (size_t)p * 3 * E;
        seq[CX_MAX_TAPS - 1 + p] = r[e] * r[2 * E + e];
    }
#pragma unroll
    for (int k = 0; k < CX_MAX_TAPS - 1; k++) {   // seq[CX_MAX_TAPS - 1 - dc + t] = memory row t
        float v = 0.0f;
#pragma unroll
        for (int t = 0; t < CX_MAX_TAPS - 1; t++)
            if (t < dc && CX_MAX_TAPS - 1 - dc + t == k) v = all[t];
        seq[k] = v;
    }
#pragma unroll
    for (int p = 0; p < CX_P; p++) {
        float u = 0.0f;
#pragma unroll
        for (int k = 0; k < CX_MAX_TAPS; k++)
            if (k <= dc) {
                float src = 0.0f;   // element p + k of [memory | bx]
#pragma unroll
                for (int s = 0; s < CX_MAX_TAPS - 1 + CX_P; s++)
                    if (s == CX_MAX_TAPS - 1 - dc + p + k) src = seq[s];
                u = fmaf(src, w[k], u);
            }
        a.u[(size_t)p * E + e] = u * a.big[(size_t)p * 3 * E + E + e];
    }
#pragma unroll
    for (int t = 0; t < CX_MAX_TAPS - 1; t++)   // new memory row t = element P + t of [memory | bx]
        if (t < dc) {
            float v = 0.0f;
#pragma unroll
            for (int s = 0; s < CX_MAX_TAPS - 1 + CX_P; s++)
                if (s == CX_MAX_TAPS - 1 - dc + CX_P + t) v = seq[s];
            a.mem[(size_t)t * E + e] = v;
        }
}

// one query head per workgroup: keys p .. p + 29 of [window | this frame] for query p, positions below 0 masked;
// q and the frame's keys rms-normed and rotated; score = fma chain over the head width / sqrtf(D); softmax with the
// max subtracted, the C library's expf and a float sum in order; o = (sum_j fma(a_j, V_j, o)) / sum * gate with
// gate = sigmoid(sum_e fma(gw_e, h_e, g)) over the layer's normed input h. The group's first head stores the
// frame's keys and values in the ring; the others read only the 29 earlier slots, which it never writes.
__global__ __launch_bounds__(CX_NT) void k_cattn(cattn_args a) {
    constexpr int W1 = CX_WIN - 1, NK = W1 + CX_P;
    __shared__ float K[NK][CX_MAX_D], V[NK][CX_MAX_D], Q[CX_P][CX_MAX_D];
    __shared__ float xs[CX_P][CX_MAX_E];
    __shared__ float gws[CX_MAX_E], l1s[CX_MAX_E];
    __shared__ float sc[CX_P][CX_WIN];
    __shared__ float sm[CX_P], gt[CX_P], hs[CX_P];
    __shared__ uint64_t cE[32];   // expf's table (an LDS copy: no memory round trip in the gate or the softmax)
    const int hh = blockIdx.x, grp = a.n_head / a.n_kv, kv = hh / grp, D = a.D, E = a.E, t = threadIdx.x;
    const int kvd = a.n_kv * D, nq = a.n_head * D, pos = a.in->pos, w = t >> 6, lane = t & 63, half = D / 2;
    const uint64_t et = kExp2Tab[t & 31];   // (requested first: its wait needs nothing later)
    for (int i = t; i < W1 * D; i += CX_NT) {
        const int j = i / D, d = i - j * D, ps = pos - W1 + j;
        float kx = 0.0f, vx = 0.0f;
        if (ps >= 0) {
            const size_t o = (size_t)(ps % CX_RING) * kvd + kv * D + d;
            kx = a.k_ring[o];
            vx = a.v_ring[o];
        }
        K[j][d] = kx;
        V[j][d] = vx;
    }
    for (int i = t; i < CX_P * D; i += CX_NT) {
        const int p = i / D, d = i - p * D;
        const float* r = a.big + (size_t)p * a.nr;
        Q[p][d] = r[hh * D + d];
        K[W1 + p][d] = r[nq + kv * D + d];
        V[W1 + p][d] = r[nq + kvd + kv * D + d];
    }
    for (int i = t; i < CX_P * E; i += CX_NT) {
        const int p = i / E, e = i - p * E;
        xs[p][e] = a.x[(size_t)p * E + e];
    }
    for (int e = t; e < E; e += CX_NT) {   // the head gate's operands, for its in-order chain
        gws[e] = a.gate_w[(size_t)hh * E + e];
        l1s[e] = a.ln1[e];
    }
    if (t < 32) cE[t] = et;
    __syncthreads();
    for (int ri = w; ri < 3 * CX_P; ri += CX_NT / 64) {   // the frame's keys, the queries, the input rows' scales
        if (ri < 2 * CX_P) {
            const int p = ri < CX_P ? ri : ri - CX_P;
            float* v = ri < CX_P ? K[W1 + p] : Q[p];
            const float* nw = ri < CX_P ? a.k_norm : a.q_norm;
            const float s = rms_scale_wave(static_cast<const float*>(v), D, a.eps);
            if (lane < half) {
                const float x0 = v[lane] * s * nw[lane], x1 = v[lane + half] * s * nw[lane + half];
                const float2 cs = a.in->cs[p][lane];
                v[lane] = fmaf(x0, cs.x, -(x1 * cs.y));
                v[lane + half] = fmaf(x0, cs.y, x1 * cs.x);
            }
        } else {
            const int p = ri - 2 * CX_P;
            const float s = rms_scale_wave(static_cast<const float*>(xs[p]), E, a.eps);
            if (lane == 0) hs[p] = s;
        }
    }
    __syncthreads();
    if (hh % grp == 0)
        for (int i = t; i < CX_P * D; i += CX_NT) {
            const int p = i / D, d = i - p * D;
            const size_t o = (size_t)((pos + p) % CX_RING) * kvd + kv * D + d;
            a.k_ring[o] = K[W1 + p][d];
            a.v_ring[o] = V[W1 + p][d];
        }
    for (int i = t; i < CX_P * CX_WIN; i += CX_NT) {
        const int p = i / CX_WIN, j = i - p * CX_WIN, kj = p + j;
        float s = -__builtin_inff();
        if (pos - W1 + kj >= 0) {
            float acc = 0.0f;
            for (int d = 0; d < D; d++) acc = fmaf(Q[p][d], K[kj][d], acc);
            s = acc / sqrtf((float)D);
        }
        sc[p][j] = s;
    }
    if (t >= 64 && t < 64 + CX_P) {   // head gate of position p (a wave the score threads leave free)
        const int p = t - 64;
        const float s = hs[p];
        float g = 0.0f;
        for (int e = 0; e < E; e++) g = fmaf(gws[e], xs[p][e] * s * l1s[e], g);
        gt[p] = 1.0f / (1.0f + expf_glibc_t(-g, cE));
    }
    __syncthreads();
    if (t < CX_P) {
        float mx = -__builtin_inff();
        for (int j = 0; j < CX_WIN; j++) mx = mx < sc[t][j] ? sc[t][j] : mx;   // std::max(mx, sc)
        float sum = 0.0f;
        for (int j = 0; j < CX_WIN; j++) {
            const float v = sc[t][j];
            const float ex = v == -__builtin_inff() ? 0.0f : expf_glibc_t(v - mx, cE);
            sc[t][j] = ex;
            sum += ex;
        }
        sm[t] = sum;
    }
    __syncthreads();
    for (int i = t; i < CX_P * D; i += CX_NT) {
        const int p = i / D, d = i - p * D;
        float acc = 0.0f;
        for (int j = 0; j < CX_WIN; j++) acc = fmaf(sc[p][j], V[p + j][d], acc);
        a.act[(size_t)p * nq + hh * D + d] = acc / sm[p] * gt[p];
    }
}

__global__ __launch_bounds__(CX_NT) void k_cresid(cresid_args a) {
    __shared__ float sc;
    const int p = blockIdx.x;
    const float* y = a.y + (size_t)p * a.E;
    float* x = a.x + (size_t)p * a.E;
    if (threadIdx.x < 64) {
        const float s = a.E == 512 ? rms_scale_wave_g<16>(y, a.eps) : rms_scale_wave(y, a.E, a.eps);
        if (threadIdx.x == 0) sc = s;
    }
    __syncthreads();
    for (int e = threadIdx.x; e < a.E; e += CX_NT) x[e] = fmaf(y[e] * sc, a.w[e], x[e]);
}

// complex products as the oracle restates imi's (the first product fused)
__device__ __forceinline__ float2 cmul(float2 a, float2 b) { return float2{fmaf(a.x, b.x, -(a.y * b.y)), fmaf(a.x, b.y, a.y * b.x)}; }
__device__ __forceinline__ float2 cadd(float2 a, float2 b) { return float2{a.x + b.x, a.y + b.y}; }
__device__ __forceinline__ float2 csub(float2 a, float2 b) { return float2{a.x - b.x, a.y - b.y}; }

// one workgroup per STFT frame p (the frames are independent until the overlap-add): the spectrum
// X_k = polar(expf(l_k), phi_k) and its conjugate mirror; the inverse DFT as imi's recursion computes it, unrolled
// into stages: the 256 five-point sums (leaf L reads elements bitrev8(L) + 256 j, j = 0 .. 4, with twiddles
// ((j k) % 5) * 256) and 8 butterfly levels (node size 1280 >> d uses twiddles k << d); the real part / n_fft
// into frames[p]
__global__ __launch_bounds__(1024) void k_cifft(cistft_args a) {
    __shared__ float2 X[CX_NFFT], O[CX_NFFT], tw[CX_NFFT];
    const int t = threadIdx.x, p = blockIdx.x;
    for (int i = t; i < CX_NFFT; i += 1024) tw[i] = a.tw[i];
    const float* lp = a.spec + (size_t)p * 2 * CX_NB;
    for (int k = t; k < CX_NB; k += 1024) {
        const float r = expf_glibc(lp[k] + a.bias[k]);
        const double ph = (double)(lp[CX_NB + k] + a.bias[CX_NB + k]);
        X[k] = float2{r * (float)cos(ph), r * (float)sin(ph)};
    }
    __syncthreads();
    for (int k = t + 1; k < CX_NB - 1; k += 1024) X[CX_NFFT - k] = float2{X[k].x, -X[k].y};
    __syncthreads();
    for (int m = t; m < CX_NFFT; m += 1024) {
        const int L = m / 5, k = m - 5 * L, off = (int)(__builtin_bitreverse32((unsigned)L) >> 24);
        float2 s = float2{0.0f, 0.0f};
#pragma unroll
        for (int j = 0; j < 5; j++) s = cadd(s, cmul(X[off + 256 * j], tw[((j * k) % 5) * 256]));
        O[m] = s;
    }
    __syncthreads();
    for (int d = 7; d >= 0; d--) {
        const int n = CX_NFFT >> d, h = n >> 1;
        if (t < CX_NFFT / 2) {
            const int node = t / h, k = t - node * h, base = node * n;
            const float2 e = O[base + k], o = cmul(O[base + k + h], tw[k << d]);
            O[base + k] = cadd(e, o);
            O[base + k + h] = csub(e, o);
        }
        __syncthreads();
    }
    for (int j = t; j < CX_NFFT; j += 1024) a.frames[(size_t)p * CX_NFFT + j] = O[j].x / (float)CX_NFFT;
}

// the overlap-add of the frame's P STFT frames in order (codec.cpp:262-269): ola += frame * hann, wsum += hann^2,
// hop samples out (ola / wsum where wsum > 1e-8), then both shifted by hop
__global__ __launch_bounds__(1024) void k_cola(cistft_args a) {
    __shared__ float hn[CX_NFFT], ol[CX_NFFT], ws[CX_NFFT];
    const int t = threadIdx.x;
    for (int i = t; i < CX_NFFT; i += 1024) {
        hn[i] = a.hann[i];
        ol[i] = a.ola[i];
        ws[i] = a.wsum[i];
    }
    __syncthreads();
    for (int p = 0; p < CX_P; p++) {
        for (int j = t; j < CX_NFFT; j += 1024) {
            ol[j] = fmaf(a.frames[(size_t)p * CX_NFFT + j], hn[j], ol[j]);
            ws[j] = fmaf(hn[j], hn[j], ws[j]);
        }
        __syncthreads();
        for (int i = t; i < CX_HOP; i += 1024) a.pcm[(size_t)p * CX_HOP + i] = ws[i] > 1e-8f ? ol[i] / ws[i] : ol[i];
        float so[2], sw[2];
#pragma unroll
        for (int r = 0; r < 2; r++) {
            const int j = t + 1024 * r, s = j + CX_HOP;
            so[r] = j < CX_NFFT && s < CX_NFFT ? ol[s] : 0.0f;
            sw[r] = j < CX_NFFT && s < CX_NFFT ? ws[s] : 0.0f;
        }
        __syncthreads();
#pragma unroll
        for (int r = 0; r < 2; r++) {
            const int j = t + 1024 * r;
            if (j < CX_NFFT) { ol[j] = so[r]; ws[j] = sw[r]; }
        }
        __syncthreads();
    }
    for (int i = t; i < CX_NFFT; i += 1024) {
        a.ola[i] = ol[i];
        a.wsum[i] = ws[i];
    }
}

}  // namespace

hipError_t launch_cfsq(const cfsq_args& a, hipStream_t s) {
    if (a.n_lvl < 1 || a.n_lvl > 16 || a.n_q < 1) return hipErrorInvalidValue;
    hipLaunchKernelGGL(k_cfsq, dim3(1), dim3(CX_NT), 0, s, a);
    return hipGetLastError();
}
hipError_t launch_crep(const crep_args& a, hipStream_t s) {
    hipLaunchKernelGGL(k_crep, dim3(((CX_P - 1) * a.E + CX_NT - 1) / CX_NT), dim3(CX_NT), 0, s, a);
    return hipGetLastError();
}
hipError_t launch_cconv(const cconv_args& a, hipStream_t s) {
    if (a.d_conv < 1 || a.d_conv > CX_MAX_TAPS - 1) return hipErrorInvalidValue;
    hipLaunchKernelGGL(k_cconv, dim3((a.E + CX_NT - 1) / CX_NT), dim3(CX_NT), 0, s, a);
    return hipGetLastError();
}
hipError_t launch_cattn(const cattn_args& a, hipStream_t s) {
    if (a.D < 32 || a.D > CX_MAX_D || a.D % 32 || a.E > CX_MAX_E || a.E % 32 || a.n_kv < 1 || a.n_head % a.n_kv)
        return hipErrorInvalidValue;
    hipLaunchKernelGGL(k_cattn, dim3(a.n_head), dim3(CX_NT), 0, s, a);
    return hipGetLastError();
}
hipError_t launch_cresid(const cresid_args& a, hipStream_t s) {
    hipLaunchKernelGGL(k_cresid, dim3(CX_P), dim3(CX_NT), 0, s, a);
    return hipGetLastError();
}
hipError_t launch_cistft(const cistft_args& a, hipStream_t s) {
    hipLaunchKernelGGL(k_cifft, dim3(CX_P), dim3(1024), 0, s, a);
    hipLaunchKernelGGL(k_cola, dim3(1), dim3(1024), 0, s, a);
    return hipGetLastError();
}

}  // namespace sh
