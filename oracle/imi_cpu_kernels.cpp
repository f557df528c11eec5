// ORACLE — test infrastructure only (see imi_cpu.h). Kernel-level restatement of imi's CPU arithmetic.
// Built with -O3 -march=native -ffp-contract=off: every fused multiply-add below is written out (fmaf or an FMA
// intrinsic) where imi's AVX2 code or GCC's default contraction of imi's scalar loops (-march=native,
// -ffp-contract=fast, imi/CMakeLists.txt:46) makes one, so the op order is fixed in the source, not by the compiler.
#include "imi_cpu.h"

#include <immintrin.h>
#include <algorithm>
#include <cmath>
#include <cstring>

namespace orc {

// imi/core/tables.cpp:20-29: sign | exponent rebias | mantissa, subnormals as m * 2^-24
float h2f(uint16_t h) {
    const uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    const uint32_t ex = (h >> 10) & 0x1fu, man = h & 0x3ffu;
    uint32_t bits;
    if (ex == 0) {
        if (man == 0) {
            bits = sign;
        } else {
            const float f = (float)man / 1024.0f / 16384.0f;
            memcpy(&bits, &f, 4);
            bits |= sign;
        }
    } else if (ex == 31) {
        bits = sign | 0x7f800000u | (man << 13);
    } else {
        bits = sign | ((ex + 112u) << 23) | (man << 13);
    }
    float f;
    memcpy(&f, &bits, 4);
    return f;
}
// imi/core/tables.cpp:30-32 (F16C, rounding mode 0 = nearest even)
uint16_t f2h(float f) { return (uint16_t)_cvtss_sh(f, 0); }

// ---- 8-row 4-bit layout (imi/core/tables.cpp:67-97) ----
bool q4_build(q4tab& t, const std::vector<const uint8_t*>& rows, int cols, bool q4_1) {
    if (rows.empty() || rows.size() % 8 || cols % 32) return false;
    t.rows = (int)rows.size(); t.cols = cols; t.nb = cols / 32; t.has_m = q4_1;
    const size_t ng = t.rows / 8, bb = q4_1 ? 20 : 18;
    t.codes.assign(ng * t.nb * 128, 0);
    t.d.assign(ng * t.nb * 8, 0);
    t.m.assign(q4_1 ? ng * t.nb * 8 : 0, 0);
    for (size_t g = 0; g < ng; g++)
        for (int j = 0; j < t.nb; j++) {
            uint8_t* c = &t.codes[(g * t.nb + j) * 128];
            for (int r = 0; r < 8; r++) {
                const uint8_t* blk = rows[8 * g + r] + (size_t)j * bb;   // fp16 d, (Q4_1: fp16 m,) 16 B of nibbles
                uint16_t d; memcpy(&d, blk, 2);
                t.d[(g * t.nb + j) * 8 + r] = d;
                if (q4_1) memcpy(&t.m[(g * t.nb + j) * 8 + r], blk + 2, 2);
                const uint8_t* qs = blk + (q4_1 ? 4 : 2);
                // file byte i holds column i (low nibble) and column 16+i (high nibble); ours keeps the byte and
                // moves it to chunk i/4, position 4r + i%4
                for (int i = 0; i < 16; i++) c[32 * (i / 4) + 4 * r + (i % 4)] = qs[i];
            }
        }
    return true;
}
// imi/core/tables.cpp:167-169
int q4_code_at(const uint8_t* c, int r, int k) {
    return k < 16 ? (c[32 * (k / 4) + 4 * r + k % 4] & 15) : (c[32 * ((k - 16) / 4) + 4 * r + (k - 16) % 4] >> 4);
}

// ---- input cut (imi/core/vec.h:47-75): elementwise ops only, so scalar == AVX2 bit for bit ----
float cut32(const float* x, int8_t* q, int* sum) {
    const __m256 sign = _mm256_set1_ps(-0.0f);
    __m256 v[4];
    __m256 mx = _mm256_setzero_ps();
    for (int k = 0; k < 4; k++) { v[k] = _mm256_loadu_ps(x + 8 * k); mx = _mm256_max_ps(mx, _mm256_andnot_ps(sign, v[k])); }
    __m128 m = _mm_max_ps(_mm256_castps256_ps128(mx), _mm256_extractf128_ps(mx, 1));
    m = _mm_max_ps(m, _mm_movehl_ps(m, m));
    m = _mm_max_ss(m, _mm_movehdup_ps(m));
    const float amax = _mm_cvtss_f32(m);
    const float d = amax / 127.0f, id = d != 0.0f ? 1.0f / d : 0.0f;
    const __m256 vid = _mm256_set1_ps(id);
    __m256i iv[4];
    for (int k = 0; k < 4; k++) iv[k] = _mm256_cvtps_epi32(_mm256_round_ps(_mm256_mul_ps(v[k], vid), _MM_FROUND_TO_NEAREST_INT | _MM_FROUND_NO_EXC));
    __m256i t = _mm256_add_epi32(_mm256_add_epi32(iv[0], iv[1]), _mm256_add_epi32(iv[2], iv[3]));
    __m128i t4 = _mm_add_epi32(_mm256_castsi256_si128(t), _mm256_extracti128_si256(t, 1));
    t4 = _mm_add_epi32(t4, _mm_shuffle_epi32(t4, 0x4e));
    t4 = _mm_add_epi32(t4, _mm_shuffle_epi32(t4, 0xb1));
    *sum = _mm_cvtsi128_si32(t4);
    // 32 x int32 -> 32 x int8 in column order (the packs interleave 128-bit halves; one dword permute restores it)
    const __m256i p = _mm256_packs_epi16(_mm256_packs_epi32(iv[0], iv[1]), _mm256_packs_epi32(iv[2], iv[3]));
    _mm256_storeu_si256((__m256i*)q, _mm256_permutevar8x32_epi32(p, _mm256_setr_epi32(0, 4, 1, 5, 2, 6, 3, 7)));
    return d;
}
void q8in::from(const float* x, int nn) {   // imi/core/tables.cpp:100-109
    n = nn;
    const int nbk = n / 32;
    if ((int)q.size() < n) { q.resize(n); d.resize(nbk); s.resize(nbk); }
    if ((int)d.size() < nbk) { d.resize(nbk); s.resize(nbk); }
    for (int j = 0; j < nbk; j++) {
        int sum;
        d[j] = cut32(x + 32 * j, &q[32 * j], &sum);
        s[j] = d[j] * (float)sum;
    }
}
void q8b::shape(int n_in, int n_cols) {      // imi/core/tables.cpp:405-409
    n = n_in; cols = n_cols; nb = cols / 32;
    if (q.size() < (size_t)n * cols) q.resize((size_t)n * cols);
    if (d.size() < (size_t)n * nb) { d.resize((size_t)n * nb); s.resize((size_t)n * nb); }
}
void q8b::set(int i, const float* x) {       // imi/core/tables.cpp:410-416
    for (int j = 0; j < nb; j++) {
        int sum;
        const float dd = cut32(x + 32 * j, &q[((size_t)j * n + i) * 32], &sum);
        d[(size_t)j * n + i] = dd;
        s[(size_t)j * n + i] = dd * (float)sum;
    }
}

// ---- Q4 x int8 block dot for 8 rows at once (imi/core/tables.cpp:115-125) ----
// chunk t of the 128-byte block holds, per row r, columns 4t..4t+3 (low nibbles) and 16+4t..16+4t+3 (high
// nibbles) at bytes 4r..4r+3; broadcasting the input's matching 4 bytes and multiplying unsigned codes by signed
// inputs puts each row's partial sum in its own 32-bit lane.
static inline __m256i block8(const uint8_t* c, const int8_t* xq) {
    const __m256i nib = _mm256_set1_epi8(15);
    __m256i acc = _mm256_setzero_si256();
    for (int t = 0; t < 4; t++) {
        int32_t lo, hi;
        memcpy(&lo, xq + 4 * t, 4);
        memcpy(&hi, xq + 16 + 4 * t, 4);
        const __m256i w = _mm256_loadu_si256((const __m256i*)(c + 32 * t));
        acc = _mm256_add_epi16(acc, _mm256_maddubs_epi16(_mm256_and_si256(w, nib), _mm256_set1_epi32(lo)));
        acc = _mm256_add_epi16(acc, _mm256_maddubs_epi16(_mm256_and_si256(_mm256_srli_epi16(w, 4), nib), _mm256_set1_epi32(hi)));
    }
    return _mm256_madd_epi16(acc, _mm256_set1_epi16(1));
}

// imi/core/tables.cpp:127-143 (Q4_0): acc = fma(float(sum), d*dx, acc); cor = fma(d, s, cor); out = acc - 8*cor
// the correction chain's per-row factor: d for Q4_0 (out = acc - 8 cor), m for Q4_1 (out = acc + cor)
// (imi/core/tables.cpp:127-143)
static inline __m256 cor_factor(const q4tab& W, const uint16_t* dp, size_t g, int j, __m256 d8) {
    return W.has_m ? _mm256_cvtph_ps(_mm_loadu_si128((const __m128i*)(W.m.data() + (g * W.nb + j) * 8))) : d8;
}
static inline __m256 q4_finish(const q4tab& W, __m256 acc, __m256 cor) {
    return W.has_m ? _mm256_add_ps(acc, cor) : _mm256_fnmadd_ps(_mm256_set1_ps(8.0f), cor, acc);
}
void q4_group(const q4tab& W, const q8in& X, int g, float* out) {
    const uint8_t* w = W.codes.data() + (size_t)g * W.nb * 128;
    const uint16_t* dp = W.d.data() + (size_t)g * W.nb * 8;
    __m256 acc = _mm256_setzero_ps(), cor = _mm256_setzero_ps();
    for (int j = 0; j < W.nb; j++) {
        const __m256i s = block8(w + (size_t)j * 128, &X.q[32 * j]);
        const __m256 d8 = _mm256_cvtph_ps(_mm_loadu_si128((const __m128i*)(dp + 8 * j)));
        acc = _mm256_fmadd_ps(_mm256_cvtepi32_ps(s), _mm256_mul_ps(d8, _mm256_set1_ps(X.d[j])), acc);
        cor = _mm256_fmadd_ps(cor_factor(W, dp, g, j, d8), _mm256_set1_ps(X.s[j]), cor);
    }
    _mm256_storeu_ps(out, q4_finish(W, acc, cor));
}
// imi/core/tables.cpp:145-163: one code load, two inputs, each accumulated exactly as q4_group
void q4_group2(const q4tab& W, const q8in& X, const q8in& X2, int g, float* out, float* out2) {
    const uint8_t* w = W.codes.data() + (size_t)g * W.nb * 128;
    const uint16_t* dp = W.d.data() + (size_t)g * W.nb * 8;
    __m256 a0 = _mm256_setzero_ps(), c0 = a0, a1 = a0, c1 = a0;
    for (int j = 0; j < W.nb; j++) {
        const uint8_t* c = w + (size_t)j * 128;
        const __m256i s0 = block8(c, &X.q[32 * j]), s1 = block8(c, &X2.q[32 * j]);
        const __m256 d8 = _mm256_cvtph_ps(_mm_loadu_si128((const __m128i*)(dp + 8 * j)));
        a0 = _mm256_fmadd_ps(_mm256_cvtepi32_ps(s0), _mm256_mul_ps(d8, _mm256_set1_ps(X.d[j])), a0);
        a1 = _mm256_fmadd_ps(_mm256_cvtepi32_ps(s1), _mm256_mul_ps(d8, _mm256_set1_ps(X2.d[j])), a1);
        const __m256 mm = cor_factor(W, dp, g, j, d8);
        c0 = _mm256_fmadd_ps(mm, _mm256_set1_ps(X.s[j]), c0);
        c1 = _mm256_fmadd_ps(mm, _mm256_set1_ps(X2.s[j]), c1);
    }
    _mm256_storeu_ps(out, q4_finish(W, a0, c0));
    _mm256_storeu_ps(out2, q4_finish(W, a1, c1));
}
// imi/core/tables.cpp:419-454: codes unpacked once per block, then every input
void q4_group_batch(const q4tab& W, const q8b& X, int g, float* out) {
    const int n = X.n, nb = W.nb;
    const __m256i nib = _mm256_set1_epi8(15), ones = _mm256_set1_epi16(1);
    __m256 acc[64], cor[64];
    for (int c = 0; c < n; c++) { acc[c] = _mm256_setzero_ps(); cor[c] = _mm256_setzero_ps(); }
    const uint8_t* w = W.codes.data() + (size_t)g * nb * 128;
    const uint16_t* dp = W.d.data() + (size_t)g * nb * 8;
    for (int j = 0; j < nb; j++) {
        __m256i lo[4], hi[4];
        for (int t = 0; t < 4; t++) {
            const __m256i v = _mm256_loadu_si256((const __m256i*)(w + (size_t)j * 128 + 32 * t));
            lo[t] = _mm256_and_si256(v, nib);
            hi[t] = _mm256_and_si256(_mm256_srli_epi16(v, 4), nib);
        }
        const __m256 d8 = _mm256_cvtph_ps(_mm_loadu_si128((const __m128i*)(dp + 8 * j)));
        const __m256 m8 = cor_factor(W, dp, g, j, d8);
        const int8_t* xq = X.q.data() + (size_t)j * n * 32;
        const float* xd = X.d.data() + (size_t)j * n;
        const float* xs = X.s.data() + (size_t)j * n;
        for (int c = 0; c < n; c++) {
            const int8_t* x = xq + 32 * c;
            __m256i a = _mm256_setzero_si256();
            for (int t = 0; t < 4; t++) {
                int32_t xa, xb;
                memcpy(&xa, x + 4 * t, 4);
                memcpy(&xb, x + 16 + 4 * t, 4);
                a = _mm256_add_epi16(a, _mm256_maddubs_epi16(lo[t], _mm256_set1_epi32(xa)));
                a = _mm256_add_epi16(a, _mm256_maddubs_epi16(hi[t], _mm256_set1_epi32(xb)));
            }
            const __m256i s = _mm256_madd_epi16(a, ones);
            acc[c] = _mm256_fmadd_ps(_mm256_cvtepi32_ps(s), _mm256_mul_ps(d8, _mm256_set1_ps(xd[c])), acc[c]);
            cor[c] = _mm256_fmadd_ps(m8, _mm256_set1_ps(xs[c]), cor[c]);
        }
    }
    for (int c = 0; c < n; c++) _mm256_storeu_ps(out + 8 * c, q4_finish(W, acc[c], cor[c]));
}
// the same arithmetic one row at a time in plain C (pins the AVX2 lane bookkeeping above)
void q4_group_scalar(const q4tab& W, const q8in& X, int g, float* out) {
    for (int r = 0; r < 8; r++) {
        float acc = 0.0f, cor = 0.0f;
        for (int j = 0; j < W.nb; j++) {
            const uint8_t* c = W.codes.data() + ((size_t)g * W.nb + j) * 128;
            int s = 0;
            for (int k = 0; k < 32; k++) s += q4_code_at(c, r, k) * X.q[32 * j + k];
            const float dd = h2f(W.d[((size_t)g * W.nb + j) * 8 + r]);
            const float mm = W.has_m ? h2f(W.m[((size_t)g * W.nb + j) * 8 + r]) : dd;
            acc = fmaf((float)s, dd * X.d[j], acc);
            cor = fmaf(mm, X.s[j], cor);
        }
        out[r] = W.has_m ? acc + cor : fmaf(-8.0f, cor, acc);
    }
}
void q4_block_sums(const q4tab& W, const q8in& X, int g, int32_t* sums) {
    for (int r = 0; r < 8; r++)
        for (int j = 0; j < W.nb; j++) {
            const uint8_t* c = W.codes.data() + ((size_t)g * W.nb + j) * 128;
            int s = 0;
            for (int k = 0; k < 32; k++) s += q4_code_at(c, r, k) * X.q[32 * j + k];
            sums[r * W.nb + j] = s;
        }
}

// ---- cfg-0 kernel (imi/kernels/q4x8.cpp) ----
void q4x8_build(q4x8tab& t, const uint8_t* w, int rows, int cols) {   // q4x8.cpp:105-119
    t.rows = rows; t.cols = cols; t.nb = cols / 32;
    const int ng = rows / 8;
    t.codes.assign((size_t)ng * t.nb * 128, 0);
    t.scales.assign((size_t)ng * t.nb * 8, 0.0f);
    auto code = [&](int r, int j, int i) {
        const uint8_t* b = w + ((size_t)r * t.nb + j) * 18;
        return i < 16 ? (b[2 + i] & 15) : (b[2 + i - 16] >> 4);
    };
    for (int g = 0; g < ng; g++)
        for (int j = 0; j < t.nb; j++) {
            uint8_t* c = &t.codes[((size_t)g * t.nb + j) * 128];
            for (int k = 0; k < 4; k++)
                for (int i = 0; i < 32; i++) c[32 * k + i] = (uint8_t)(code(8 * g + 2 * k, j, i) | (code(8 * g + 2 * k + 1, j, i) << 4));
            for (int r = 0; r < 8; r++) {
                uint16_t d; memcpy(&d, w + ((size_t)(8 * g + r) * t.nb + j) * 18, 2);
                t.scales[((size_t)g * t.nb + j) * 8 + r] = h2f(d);
            }
        }
}
void q4x8_quant_in(const float* x, int n, q4x8in& o) {   // q4x8.cpp:38-48: roundf (half away from zero)
    const int nb = n / 32;
    o.q.resize(n); o.d.resize(nb); o.corr.resize(nb);
    for (int j = 0; j < nb; j++) {
        float amax = 0.0f;
        for (int i = 0; i < 32; i++) amax = std::max(amax, fabsf(x[32 * j + i]));
        const float d = amax / 127.0f, id = d != 0.0f ? 1.0f / d : 0.0f;
        int s = 0;
        for (int i = 0; i < 32; i++) { const int v = (int)roundf(x[32 * j + i] * id); o.q[32 * j + i] = (int8_t)v; s += v; }
        o.d[j] = d;
        o.corr[j] = 8.0f * d * (float)s;
    }
}
// q4x8.cpp:51-77. Integer row sums are order-free; the fp32 epilogue: acc = fma(float(s), d*dx, acc),
// cor = fma(d, corr, cor), y = acc - cor.
void q4x8_rows(const q4x8tab& W, const q4x8in& X, float* y, int g0, int g1) {
    const int nb = W.nb;
    const __m256i nib = _mm256_set1_epi8(15), ones = _mm256_set1_epi16(1);
    for (int g = g0; g < g1; g++) {
        const uint8_t* w = &W.codes[(size_t)g * nb * 128];
        const float* sc = &W.scales[(size_t)g * nb * 8];
        __m256 acc = _mm256_setzero_ps(), cor = _mm256_setzero_ps();
        for (int j = 0; j < nb; j++) {
            const uint8_t* c = w + (size_t)j * 128;
            // chunk k holds rows 2k (low nibbles) and 2k+1 (high nibbles), byte i = column i; each row's 32
            // products reduce to 8 dword partials, and a pairwise-add tree folds the 8 rows into one register
            const __m256i xv = _mm256_loadu_si256((const __m256i*)&X.q[32 * j]);
            __m256i p[8];
            for (int k = 0; k < 4; k++) {
                const __m256i v = _mm256_loadu_si256((const __m256i*)(c + 32 * k));
                p[2 * k] = _mm256_madd_epi16(_mm256_maddubs_epi16(_mm256_and_si256(v, nib), xv), ones);
                p[2 * k + 1] = _mm256_madd_epi16(_mm256_maddubs_epi16(_mm256_and_si256(_mm256_srli_epi16(v, 4), nib), xv), ones);
            }
            const __m256i q01 = _mm256_hadd_epi32(p[0], p[1]), q23 = _mm256_hadd_epi32(p[2], p[3]);
            const __m256i q45 = _mm256_hadd_epi32(p[4], p[5]), q67 = _mm256_hadd_epi32(p[6], p[7]);
            const __m256i qa = _mm256_hadd_epi32(q01, q23), qb = _mm256_hadd_epi32(q45, q67);
            const __m256i ssum = _mm256_add_epi32(_mm256_permute2x128_si256(qa, qb, 0x20), _mm256_permute2x128_si256(qa, qb, 0x31));
            const __m256 d8 = _mm256_loadu_ps(sc + (size_t)j * 8);
            acc = _mm256_fmadd_ps(_mm256_cvtepi32_ps(ssum), _mm256_mul_ps(d8, _mm256_set1_ps(X.d[j])), acc);
            cor = _mm256_fmadd_ps(d8, _mm256_set1_ps(X.corr[j]), cor);
        }
        _mm256_storeu_ps(y + 8 * g, _mm256_sub_ps(acc, cor));
    }
}

// ---- Q8_0 k-major tables (imi/core/tables.cpp:289-318) ----
void q8_0_dequant_row(const uint8_t* row, float* y, int cols) {   // tables.cpp:292-295
    for (int j = 0; j < cols / 32; j++) {
        uint16_t dh; memcpy(&dh, row + 34 * j, 2);
        const float d = h2f(dh);
        const int8_t* qs = (const int8_t*)(row + 34 * j + 2);
        for (int i = 0; i < 32; i++) y[32 * j + i] = d * (float)qs[i];
    }
}
// ---- Q6_K word table ----
// imi/core/tables.cpp:200-213: per 256 values amax, d = amax / 127, codes lrintf(v / d) (half-even), and the code sum
// of every 16 values as int16
void q8kin::from(const float* x, int nn) {
    n = nn;
    const int nbk = n / 256;
    q.resize(n); d.resize(nbk); bsums.resize((size_t)nbk * 16);
    for (int j = 0; j < nbk; j++) {
        const float* v = x + 256 * j;
        float amax = 0.0f;
        for (int i = 0; i < 256; i++) amax = std::max(amax, fabsf(v[i]));
        d[j] = amax / 127.0f;
        const float id = d[j] != 0.0f ? 1.0f / d[j] : 0.0f;
        int8_t* c = &q[256 * j];
        for (int s = 0; s < 16; s++) {
            int t = 0;
            for (int i = 16 * s; i < 16 * s + 16; i++) t += (c[i] = (int8_t)lrintf(v[i] * id));
            bsums[16 * j + s] = (int16_t)t;
        }
    }
}
// value e of a Q6_K block: e = 128 h + 32 k + l; low 4 bits from ql[64 h + 32 (k & 1) + l] (low nibble for k < 2,
// high nibble for k >= 2), high 2 bits from bits 2k, 2k+1 of qh[32 h + l] (imi/core/tables.cpp:219-230)
int q6k_at(const uint8_t* blk, int e) {
    const int h = e >> 7, k = (e >> 5) & 3, l = e & 31;
    const uint8_t lo = blk[64 * h + 32 * (k & 1) + l], hi = blk[128 + 32 * h + l];
    return ((k < 2 ? lo : lo >> 4) & 15) | (((hi >> (2 * k)) & 3) << 4);
}
static float blk_d(const uint8_t* blk) { uint16_t dh; memcpy(&dh, blk + 208, 2); return h2f(dh); }
// y = d * scale[e / 16] * (value - 32), the two products in that order (imi/core/tables.cpp:216-233)
void q6k_dequant_row(const uint8_t* row, float* y, int nblocks) {
    for (int i = 0; i < nblocks; i++) {
        const uint8_t* b = row + 210 * (size_t)i;
        const float d = blk_d(b);
        const int8_t* sc = (const int8_t*)(b + 192);
        for (int e = 0; e < 256; e++) y[256 * i + e] = d * (float)sc[e >> 4] * (float)(q6k_at(b, e) - 32);
    }
}
// imi/core/tables.cpp:246-270, lane by lane. Per 128-value half h and 32-value chunk k, maddubs pairs bytes and madd
// pairs those, so int32 lane l takes values 4l .. 4l+3 of the chunk, weighted by the chunk's scale for its half of
// the register (lanes 0-3: scale 8h + 2k, lanes 4-7: 8h + 2k + 1); corr lane l = sc[2l] bsums[2l] + sc[2l+1]
// bsums[2l+1], and each lane ends as sum - 32 corr. Integer, exact.
void q6k_lane_sums(const uint8_t* blk, const q8kin& X, int i, int32_t out[8]) {
    const int8_t* sc = (const int8_t*)(blk + 192);
    const int8_t* xq = &X.q[256 * (size_t)i];
    const int16_t* bs = &X.bsums[16 * (size_t)i];
    for (int l = 0; l < 8; l++) {
        int32_t s = 0;
        for (int h = 0; h < 2; h++)
            for (int k = 0; k < 4; k++) {
                int32_t p = 0;
                for (int u = 0; u < 4; u++) {
                    const int e = 128 * h + 32 * k + 4 * l + u;
                    p += q6k_at(blk, e) * xq[e];
                }
                s += p * sc[8 * h + 2 * k + (l >> 2)];
            }
        const int32_t corr = sc[2 * l] * bs[2 * l] + sc[2 * l + 1] * bs[2 * l + 1];
        out[l] = s - 32 * corr;
    }
}
// imi/core/tables.cpp:271-276: acc_l = fma(d * X.d[i], float(lane_l), acc_l) over blocks; then the 256-bit
// horizontal sum ((a0 + a4) + (a2 + a6)) + ((a1 + a5) + (a3 + a7))
float q6k_row(const uint8_t* row, const q8kin& X, int nblocks) {
    float acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    for (int i = 0; i < nblocks; i++) {
        const uint8_t* b = row + 210 * (size_t)i;
        int32_t lane[8];
        q6k_lane_sums(b, X, i, lane);
        const float dd = blk_d(b) * X.d[i];
        for (int l = 0; l < 8; l++) acc[l] = fmaf(dd, (float)lane[l], acc[l]);
    }
    return ((acc[0] + acc[4]) + (acc[2] + acc[6])) + ((acc[1] + acc[5]) + (acc[3] + acc[7]));
}

bool q8g_build(q8gtab& t, const std::vector<const uint8_t*>& rows, int cols) {
    if (rows.empty() || cols % 32) return false;
    t.rows = (int)rows.size(); t.rows_pad = (t.rows + 7) / 8 * 8; t.cols = cols; t.nb = cols / 32;
    const size_t ng = t.rows_pad / 8;
    t.codes.assign(ng * cols * 8, 0);
    t.d.assign(ng * t.nb * 8, 0);
    for (int r = 0; r < t.rows; r++) {
        const size_t g = r / 8, rr = r % 8;
        for (int j = 0; j < t.nb; j++) {
            const uint8_t* b = rows[r] + (size_t)j * 34;
            uint16_t dh; memcpy(&dh, b, 2);
            t.d[(g * t.nb + j) * 8 + rr] = dh;
            for (int i = 0; i < 32; i++) t.codes[(g * cols + 32 * j + i) * 8 + rr] = (int8_t)b[2 + i];
        }
    }
    return true;
}
// imi/core/tables.cpp:385-402. C = 1 takes the AVX2 one-input path (:366-382): four chains over columns
// kk % 4, each a_i = fma(float(w), d*x, a_i), then (a0+a1)+(a2+a3). C = 12 / 6 take the multi-input paths
// (:324-365): w*d once per column, then a_c = fma(wd, x_c, a_c). Any other C takes the generic path: per block and
// row, s = sum over 32 columns of fma(float(w), x, s), then acc += d*s (contracted by GCC to fma(d, s, acc)).
void q8g_group(const q8gtab& W, const float* xt, int C, int g, float* out) {
    const int8_t* w = W.codes.data() + (size_t)g * W.cols * 8;
    const uint16_t* dp = W.d.data() + (size_t)g * W.nb * 8;
    if (C == 1) {
        __m256 a0 = _mm256_setzero_ps(), a1 = a0, a2 = a0, a3 = a0;
        for (int j = 0; j < W.nb; j++) {
            const __m256 d8 = _mm256_cvtph_ps(_mm_loadu_si128((const __m128i*)(dp + 8 * j)));
            const int8_t* wj = w + (size_t)j * 256;
            const float* xj = xt + 32 * j;
            for (int kk = 0; kk < 32; kk += 4) {
                auto wv = [&](int o) { return _mm256_cvtepi32_ps(_mm256_cvtepi8_epi32(_mm_loadl_epi64((const __m128i*)(wj + (kk + o) * 8)))); };
                a0 = _mm256_fmadd_ps(wv(0), _mm256_mul_ps(d8, _mm256_set1_ps(xj[kk])), a0);
                a1 = _mm256_fmadd_ps(wv(1), _mm256_mul_ps(d8, _mm256_set1_ps(xj[kk + 1])), a1);
                a2 = _mm256_fmadd_ps(wv(2), _mm256_mul_ps(d8, _mm256_set1_ps(xj[kk + 2])), a2);
                a3 = _mm256_fmadd_ps(wv(3), _mm256_mul_ps(d8, _mm256_set1_ps(xj[kk + 3])), a3);
            }
        }
        _mm256_storeu_ps(out, _mm256_add_ps(_mm256_add_ps(a0, a1), _mm256_add_ps(a2, a3)));
        return;
    }
    if (C == 12 || C == 6) {
        std::vector<__m256> a(C, _mm256_setzero_ps());
        for (int j = 0; j < W.nb; j++) {
            const __m256 d8 = _mm256_cvtph_ps(_mm_loadu_si128((const __m128i*)(dp + 8 * j)));
            const int8_t* wj = w + (size_t)j * 256;
            const float* xj = xt + (size_t)j * 32 * C;
            for (int kk = 0; kk < 32; kk++) {
                const __m256 wv = _mm256_mul_ps(_mm256_cvtepi32_ps(_mm256_cvtepi8_epi32(_mm_loadl_epi64((const __m128i*)(wj + kk * 8)))), d8);
                for (int c = 0; c < C; c++) a[c] = _mm256_fmadd_ps(wv, _mm256_set1_ps(xj[kk * C + c]), a[c]);
            }
        }
        for (int c = 0; c < C; c++) _mm256_storeu_ps(out + 8 * c, a[c]);
        return;
    }
    std::vector<float> acc((size_t)C * 8, 0.0f);
    for (int j = 0; j < W.nb; j++)
        for (int r = 0; r < 8; r++) {
            const float dd = h2f(dp[8 * j + r]);
            for (int c = 0; c < C; c++) {
                float s = 0.0f;
                for (int kk = 0; kk < 32; kk++) {
                    const int k = 32 * j + kk;
                    s = fmaf((float)w[(size_t)k * 8 + r], xt[(size_t)k * C + c], s);
                }
                acc[(size_t)c * 8 + r] = fmaf(dd, s, acc[(size_t)c * 8 + r]);
            }
        }
    memcpy(out, acc.data(), acc.size() * sizeof(float));
}

// ---- small vector math ----
// imi/core/vec.h:20-33: four 8-lane FMA accumulators over 32-column strides, (a0+a1)+(a2+a3), then the
// 8-lane horizontal sum ((l0+l4)+(l2+l6)) + ((l1+l5)+(l3+l7))
float rms_scale(const float* x, int n, float eps) {
    __m256 a0 = _mm256_setzero_ps(), a1 = a0, a2 = a0, a3 = a0;
    for (int i = 0; i < n; i += 32) {
        const __m256 v0 = _mm256_loadu_ps(x + i), v1 = _mm256_loadu_ps(x + i + 8), v2 = _mm256_loadu_ps(x + i + 16), v3 = _mm256_loadu_ps(x + i + 24);
        a0 = _mm256_fmadd_ps(v0, v0, a0); a1 = _mm256_fmadd_ps(v1, v1, a1);
        a2 = _mm256_fmadd_ps(v2, v2, a2); a3 = _mm256_fmadd_ps(v3, v3, a3);
    }
    const __m256 v = _mm256_add_ps(_mm256_add_ps(a0, a1), _mm256_add_ps(a2, a3));
    __m128 r = _mm_add_ps(_mm256_castps256_ps128(v), _mm256_extractf128_ps(v, 1));
    r = _mm_add_ps(r, _mm_movehl_ps(r, r));
    r = _mm_add_ss(r, _mm_movehdup_ps(r));
    const float s = _mm_cvtss_f32(r);
    return 1.0f / sqrtf(s / (float)n + eps);
}
void norm_mul(const float* x, const float* w, float* o, int n, float eps) {   // vec.h:36-39
    const float sc = rms_scale(x, n, eps);
    for (int i = 0; i < n; i++) o[i] = x[i] * sc * w[i];
}
void norm_mul_add(const float* y, const float* w, float* x, int n, float eps) {   // vec.h:41-44, contracted add
    const float sc = rms_scale(y, n, eps);
    for (int i = 0; i < n; i++) x[i] = fmaf(y[i] * sc, w[i], x[i]);
}
// imi/core/seoul.cpp:19-28: th starts at pos and is multiplied by base^(-2/n) per pair; GCC contracts the
// rotation's first product into the subtraction/addition
void rope(float* v, int n, int pos, float base, const float* ff) {
    const float scale = powf(base, -2.0f / (float)n);
    float th = (float)pos;
    for (int i = 0; i < n / 2; i++) {
        const float a = th / (ff ? ff[i] : 1.0f), c = cosf(a), s = sinf(a);
        const float x0 = v[i], x1 = v[i + n / 2];
        v[i] = fmaf(x0, c, -(x1 * s));
        v[i + n / 2] = fmaf(x0, s, x1 * c);
        th *= scale;
    }
}
// seoul.cpp:29-39: 8-lane FMA accumulator, then the 8-lane horizontal sum
float dot_h(const float* q, const uint16_t* k, int n) {
    __m256 a = _mm256_setzero_ps();
    for (int i = 0; i < n; i += 8) a = _mm256_fmadd_ps(_mm256_loadu_ps(q + i), _mm256_cvtph_ps(_mm_loadu_si128((const __m128i*)(k + i))), a);
    __m128 r = _mm_add_ps(_mm256_castps256_ps128(a), _mm256_extractf128_ps(a, 1));
    r = _mm_add_ps(r, _mm_movehl_ps(r, r));
    r = _mm_add_ss(r, _mm_movehdup_ps(r));
    return _mm_cvtss_f32(r);
}
void axpy_h(float p, const uint16_t* v, float* o, int n) {   // seoul.cpp:40-47
    const __m256 pp = _mm256_set1_ps(p);
    for (int i = 0; i < n; i += 8)
        _mm256_storeu_ps(o + i, _mm256_fmadd_ps(pp, _mm256_cvtph_ps(_mm_loadu_si128((const __m128i*)(v + i))), _mm256_loadu_ps(o + i)));
}

}  // namespace orc
