// The ears on the device (imi/core/ears.{h,cpp}): 16 kHz samples -> [positions][n_out] rows for the brain's
// prefill. Kernel arguments and launchers.
//
// Layouts: float tables as [cols / 8][rows_pad][8] (F16 bits or F32; element (r, k) at ((k / 8) rows_pad + r) 8 +
// k % 8, so a wave's 64 rows read 1 KB per 8 columns); table inputs feature-major [cols][ldx] (positions contiguous,
// ldx a multiple of 4); the residual stream and the layer's q|k|v or b|c|x rows position-major [P][width].
#pragma once
#include <hip/hip_runtime.h>

#include <cstdint>

namespace sh {

constexpr int EA_NP = 4;          // positions per table thread (wave-uniform)
constexpr int EA_MAX_WIN = 64;    // attention window the kernel takes (one lane per key)
constexpr int EA_MAX_D = 128;

enum ea_epi : int {
    EE_STORE = 0,   // acc + bias (or + 0)
    EE_ADD = 1,     // out + (acc + 0): the residual add of imi's table(..., add = true)
    EE_SILU = 2,    // silu(acc + bias)
    EE_GELU = 3,    // gelu_erf(acc + bias)
    EE_GLU = 4,     // (gate, up) groups of 8 rows: silu(gate) * up into row 8 q + r
    EE_POWER = 5,   // (cos, -sin) row pairs: re * re + im * im into row b
};

struct etab {
    const void* w = nullptr;
    int rows = 0, rows_pad = 0, cols = 0;
    bool f32 = false;
};

struct etab_args {
    etab W;
    const float* x;     // [cols][ldx]
    int ldx, P;         // P: positions computed and stored (ldx >= P rounded up to 4)
    const float* bias;  // [rows] or null
    float* out;
    int ldo;
    bool xt_out;        // out feature-major [rows'][ldo] (else position-major [P][ldo])
};

hipError_t launch_etab(int epi, const etab_args& a, hipStream_t s);

// fx[k][fr] = hann[k] * pcm[fr * hop + k] (0 past the clip or past n_fr), k < n_fft, fr < ldf
hipError_t launch_eframes(const float* pcm, int n, const float* hann, int n_fft, int hop, int n_fr, float* fx, int ldf,
                          hipStream_t s);
// mel[fr][m] = (log10(max(sum_b fb[m][b] pw[b][fr], 1e-12)) + 4) / 4, the sum an fma chain in double over the
// filter's nonzero bins span[m] = [lo, hi)
hipError_t launch_emel(const float* pw, int ldp, const float* fb, const int2* span, int n_bin, int n_mel, int n_fr,
                       float* mel, hipStream_t s);
// first stride-2 3x3 conv of the mel image (one input channel) + SiLU: a0[c][t][f], t < T2, f < F2
hipError_t launch_econv0(const float* mel, int n_fr, int n_mel, const float* w9, const float* b, int C, float* a0,
                         hipStream_t s);
// depthwise stride-2 3x3 conv: in[c][Ti][Fi] (channel stride ldi) -> out[c][To][Fo] (channel stride ldo)
hipError_t launch_edw(const float* in, int Ti, int Fi, int ldi, const float* w9, const float* b, int C, float* out,
                      int ldo, hipStream_t s);
// xf[(c F8 + f)][p] = a[c][p F8 + f] for p < P (zero for P <= p < ldf)
hipError_t launch_eflat(const float* a, int lda, int C, int F8, int P, float* xf, int ldf, hipStream_t s);
// h[e][p] = x[p][e] * rms(x[p]) * w[e] (imi_norm_mul), zero for P <= p < ldh
hipError_t launch_enorm(const float* x, const float* w, int E, int P, float eps, float* h, int ldh, hipStream_t s);
// short conv of a layer: act[e][p] = c[p][e] * sum_k fma(w[k][e], b[t][e] * x[t][e], .), t = p - (d - 1) + k >= 0
hipError_t launch_econv(const float* big, int ld, const float* w, int E, int d_conv, int P, float* act, int lda,
                        hipStream_t s);
// q and k of every position and head: norm times weight, then rope with the host's (cos, sin) rows cs[p][D / 2]
hipError_t launch_eqk(float* big, int ld, int n_head, int n_kv, int D, const float* q_norm, const float* k_norm,
                      const float2* cs, int P, float eps, hipStream_t s);
// attention of each (position, head) over the last `window` positions: act[h D + i][p]
hipError_t launch_eattn(const float* big, int ld, int n_head, int n_kv, int D, int window, int P, float* act, int lda,
                        hipStream_t s);
// last norm, then LayerNorm with double mean and variance: h[e][p]
hipError_t launch_efinal(const float* x, const float* post_ln, const float* ln_w, const float* ln_b, int E, int P,
                         float eps, float* h, int ldh, hipStream_t s);

}  // namespace sh
