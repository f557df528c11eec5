// The codec decoder on the device (imi/core/codec.{h,cpp}): codes -> 24 kHz samples. Kernel arguments and launchers;
// the table products reuse the voice generator's Q8_0 kernels (imi_q8g_group's operation orders).
#pragma once
#include <hip/hip_runtime.h>

#include <cstdint>

namespace sh {

constexpr int CX_P = 6;          // positions (STFT frames) per codec frame (imi/core/codec.h:34)
constexpr int CX_WIN = 30;       // attention window, this position included
constexpr int CX_RING = 36;      // key/value ring slots: the 29 earlier positions and this frame's 6 never share one
constexpr int CX_NFFT = 1280;    // inverse FFT size: 2^8 x 5
constexpr int CX_HOP = 320;
constexpr int CX_NB = 641;       // frequency bins
constexpr int CX_NCB = 12;       // codes per frame
constexpr int CX_MAX_D = 128;    // head width the kernels take
constexpr int CX_MAX_TAPS = 8;   // conv taps (memory rows + 1)

// what the host writes before each frame (pinned, one copy)
struct cframe_in {
    int32_t codes[CX_NCB];
    int32_t pos;                                // position of the frame's first STFT frame
    float2 cs[CX_P][CX_MAX_D / 2];              // rope (cos, sin) of positions pos .. pos + 5, pair i
};

// codes -> FSQ levels -> quantizer projection (imi/core/codec.cpp:147-152)
struct cfsq_args {
    const cframe_in* in;
    const float* lvl;        // [n_codes][n_lvl]
    const float* w;          // [n_q][n_cb * n_lvl]
    const float* b;          // [n_q]
    int n_lvl, n_q;
    float* out;              // [n_q]
};

// x[p] = x[0] for p = 1 .. 5 (nearest upsampling, codec.cpp:158)
struct crep_args { float* x; int E; };

// gated short conv over [memory | this frame] (codec.cpp:166-191): big [P][3E] = (b, c, x) rows
struct cconv_args {
    const float* big;
    const float* taps;       // [d_conv + 1][E]
    float* mem;              // [d_conv][E] carried memory, updated in place (each thread owns its channel)
    float* u;                // [P][E]
    int E, d_conv;
};

// gated attention of one query head over the window (codec.cpp:193-236)
struct cattn_args {
    const cframe_in* in;
    const float* big;        // [P][nr]: q (H D) | k (Hk D) | v (Hk D), this frame's rows
    int nr;
    const float* x;          // [P][E] the layer input (its ln1 norm feeds the head gates)
    const float* ln1;
    const float* gate_w;     // [H][E]
    const float* q_norm;
    const float* k_norm;
    float* k_ring;           // [CX_RING][Hk D] normed, rotated keys by position % CX_RING
    float* v_ring;
    float* act;              // [P][H D]
    int E, n_head, n_kv, D;
    float eps;
};

// x[p] = fma(y[p] * rms(y[p]), w, x[p]) (imi_norm_mul_add, codec.cpp:237,250)
struct cresid_args { const float* y; const float* w; float* x; int E; float eps; };

// log magnitudes and phases -> inverse FFT -> overlap-add of the frame's 6 STFT frames (codec.cpp:254-269)
struct cistft_args {
    const float* spec;       // [P][2 nb] out_proj rows before the bias
    const float* bias;       // [2 nb]
    const float2* tw;        // [n_fft] polar(1, 2 pi i / n_fft), as the host's C library makes them
    const float* hann;       // [n_fft]
    float* ola;              // [n_fft] carried
    float* wsum;             // [n_fft] carried
    float* pcm;              // [P][hop] samples before the start trim
    float* frames;           // [P][n_fft] work: each STFT frame's inverse transform, real part / n_fft
};

hipError_t launch_cfsq(const cfsq_args& a, hipStream_t s);
hipError_t launch_crep(const crep_args& a, hipStream_t s);
hipError_t launch_cconv(const cconv_args& a, hipStream_t s);
hipError_t launch_cattn(const cattn_args& a, hipStream_t s);
hipError_t launch_cresid(const cresid_args& a, hipStream_t s);
hipError_t launch_cistft(const cistft_args& a, hipStream_t s);

}  // namespace sh
