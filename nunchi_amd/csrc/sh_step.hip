// The persistent step kernel (gfx950, wave64): one 512-thread workgroup per compute unit, all co-resident
// (cooperative launch), running n decode steps of imi's brain (imi/core/seoul.cpp:359-488) without returning to the
// host.
//
// Work split. Every table read is split by 8-row groups across the workgroups (contiguous unit ranges, fixed for the
// whole launch, so a workgroup always owns the same rows, conv channels and attention heads). Inside a workgroup a
// chunk of at most 512 (group, block) pairs is computed as in the decode GEMV: phase 1, one pair per thread, loads
// the 8 rows' 16-byte code blocks and the group's scales and forms the exact integer dots against the int8-cut
// input; phase 2 runs imi's per-row fp32 chains over the blocks in order (imi/core/tables.cpp:127-143), the
// acc chains and the cor chains on different waves. The arithmetic is the CPU's, op for op.
//
// Synchronisation. A stage's outputs are published as 8-byte records {value, tag} with device-scope stores; the
// tag is the step's epoch. Consumers load the records with device-scope loads and wait until every tag they need
// is current: no grid barrier, no fences, and the wait is one memory round trip after the last producer's store.
// Buffers alternate by epoch parity, so a record is never overwritten while a slower workgroup may still read it.
// Every wait gives up after `timeout` wall-clock ticks and raises `err`, and every workgroup then leaves.
//
// Prefetch. Each thread holds two register sets of one pair's weights (9 x 16 B). Before a chunk is computed, the
// loads of this workgroup's next chunk are issued into the other set, so the stream of the next stage's weights is
// in flight while the workgroup waits for that stage's input.
//
// Address spaces are explicit: weights, records, caches as global (1), LDS as local (3), the stage table as
// constant (4). Generic (flat) accesses would count against the LDS wait counter as well and tie every LDS wait to
// the outstanding weight prefetch.
#include <hip/hip_runtime.h>

#include "sh_device.h"
#include "sh_step.h"

namespace sh {
namespace {

typedef unsigned long long u64;
#define GLB __attribute__((address_space(1)))
#define LDS __attribute__((address_space(3)))
#define CST __attribute__((address_space(4)))
typedef const sk_stage CST& SR;
typedef float f32x2 __attribute__((ext_vector_type(2)));

__device__ __forceinline__ void ll_put(u64* p, float v, unsigned tag) {
    const u64 r = ((u64)tag << 32) | (u64)__float_as_uint(v);
    __hip_atomic_store((u64 GLB*)p, r, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ u64 ll_load(const u64* p) {
    return __hip_atomic_load((u64 GLB*)const_cast<u64*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// wait for the record at p to carry tag; false after the timeout or when another workgroup gave up
__device__ __forceinline__ bool ll_wait(const u64* p, unsigned tag, float* v, const sk_params& P) {
    u64 r = ll_load(p);
    if ((unsigned)(r >> 32) != tag) {
        const long long t0 = wall_clock64();
        for (;;) {
            __builtin_amdgcn_s_sleep(1);
            r = ll_load(p);
            if ((unsigned)(r >> 32) == tag) break;
            if (wall_clock64() - t0 > P.timeout || __hip_atomic_load((int GLB*)P.err, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) != 0) {
                __hip_atomic_store((int GLB*)P.err, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                return false;
            }
        }
    }
    *v = __uint_as_float((unsigned)r);
    return true;
}

// n_m x n_per records, value (m, i) = src[m * src_ld + i] -> dst[m * dst_ld + i]. Each thread loads up to 16 of
// its records at once and reloads together those whose tag is not yet current, so the wait costs one memory round
// trip after the last producer's store, not one per record.
template <class DST>
__device__ __forceinline__ bool ll_gather(const u64* src, int src_ld, int n_per, int n_m, unsigned tag, DST dst, int dst_ld,
                                          const sk_params& P) {
    constexpr int B = 8;
    const int per_m = (n_per + SK_THREADS - 1) / SK_THREADS;   // records of one conversation per thread
    const int n_tot = n_m * per_m;                              // this thread's record slots
    for (int q0 = 0; q0 < n_tot; q0 += B) {
        u64 r[B];
        int off[B];   // record offset from src, or -1
#pragma unroll
        for (int q = 0; q < B; q++) {
            const int k = q0 + q, m = k / per_m, i = (k - m * per_m) * SK_THREADS + (int)threadIdx.x;
            off[q] = (k < n_tot && i < n_per) ? m * src_ld + i : -1;
            r[q] = off[q] >= 0 ? ll_load(src + off[q]) : ((u64)tag << 32);
        }
        long long t0 = 0;
        for (;;) {
            bool all = true;
#pragma unroll
            for (int q = 0; q < B; q++) all &= (unsigned)(r[q] >> 32) == tag;
            if (all) break;
            if (t0 == 0) t0 = wall_clock64();
            if (wall_clock64() - t0 > P.timeout || __hip_atomic_load((int GLB*)P.err, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) != 0) {
                __hip_atomic_store((int GLB*)P.err, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                return false;
            }
            __builtin_amdgcn_s_sleep(1);
#pragma unroll
            for (int q = 0; q < B; q++)
                if ((unsigned)(r[q] >> 32) != tag) r[q] = ll_load(src + off[q]);
        }
#pragma unroll
        for (int q = 0; q < B; q++)
            if (off[q] >= 0) {
                const int m = off[q] / src_ld, i = off[q] - m * src_ld;
                dst[m * dst_ld + i] = __uint_as_float((unsigned)r[q]);
            }
    }
    return true;
}

// ---------------------------------------------------------------- LDS map
__device__ __forceinline__ char LDS* lds_base() {
    extern __shared__ __align__(16) char smem_dyn[];
    return (char LDS*)smem_dyn;
}
__device__ __forceinline__ float LDS* l_x() { return (float LDS*)(lds_base() + SK_OFF_X); }      // [2][32][68]
__device__ __forceinline__ float LDS* l_y() { return (float LDS*)(lds_base() + SK_OFF_Y); }      // [2][32][68]
__device__ __forceinline__ int LDS* l_xq() { return (int LDS*)(lds_base() + SK_OFF_XQ); }        // [2][2048] int8 x 4
__device__ __forceinline__ float LDS* l_dx() { return (float LDS*)(lds_base() + SK_OFF_DX); }    // [2][256]
__device__ __forceinline__ float LDS* l_s() { return (float LDS*)(lds_base() + SK_OFF_S); }      // [2][256]
__device__ __forceinline__ float LDS* l_pq() { return (float LDS*)(lds_base() + SK_OFF_OPS); }  // [2][M][rows][st]
__device__ __forceinline__ float LDS* l_stg() { return (float LDS*)(lds_base() + SK_OFF_OPS); }  // [2][8192] staging
__device__ __forceinline__ float LDS* l_dd() { return (float LDS*)(lds_base() + SK_OFF_DD); }    // [rows][nb + 4]
__device__ __forceinline__ float LDS* l_cor() { return (float LDS*)(lds_base() + SK_OFF_COR); }  // [256]
__device__ __forceinline__ float LDS* l_out() { return (float LDS*)(lds_base() + SK_OFF_OUT); }  // [256]
__device__ __forceinline__ float LDS* l_redv() { return (float LDS*)(lds_base() + SK_OFF_RED); } // [512]
__device__ __forceinline__ int LDS* l_redi() { return (int LDS*)(lds_base() + SK_OFF_RED + 2048); }
__device__ __forceinline__ float LDS* l_misc() { return (float LDS*)(lds_base() + SK_OFF_MISC); } // [32]
__device__ __forceinline__ int LDS* l_misci() { return (int LDS*)(lds_base() + SK_OFF_MISC + 128); }
__device__ __forceinline__ float LDS* l_att() { return (float LDS*)(lds_base() + SK_OFF_OPS); }  // attention's share

// ---------------------------------------------------------------- work split
struct wg_range {
    int u0, n, cu, nch;
};
typedef int i32x4 __attribute__((ext_vector_type(4)));
__device__ __forceinline__ i32x4 LDS* l_rng() { return (i32x4 LDS*)(lds_base() + SK_OFF_RNG); }

// this workgroup's contiguous units of stage S and their chunking (units per chunk cu, chunks nch); computed once
// per launch into LDS, read from there afterwards
template <int M>
__device__ __forceinline__ wg_range compute_range(SR S, int b, int G) {
    wg_range r;
    const unsigned U = (unsigned)S.units;
    r.u0 = (int)((U * (unsigned)b) / (unsigned)G);
    r.n = (int)((U * (unsigned)(b + 1)) / (unsigned)G) - r.u0;
    const int nb = S.W.nb > 0 ? S.W.nb : 1;
    r.cu = max(1, sk_gmax(nb, M) / max(S.ug, 1));
    r.nch = S.kind == SK_ATTN ? 0 : (r.n + r.cu - 1) / r.cu;
    return r;
}
__device__ __forceinline__ wg_range range_at(int s) {
    const i32x4 v = l_rng()[s];
    return wg_range{v.x, v.y, v.z, v.w};
}

__device__ __forceinline__ SR stage_at(const sk_params& P, int k) { return ((const sk_stage CST*)P.stages)[k]; }

// the workgroup's chunks of one step in walk order, built once per launch: entry = stage | chunk << 8 | vocab << 16;
// word 0 holds the count
__device__ __forceinline__ int LDS* l_cl() { return (int LDS*)(lds_base() + SK_OFF_CL); }
constexpr int SK_CL_VOCAB = 1 << 16;

template <int M>
__device__ __forceinline__ void build_chunk_list(const sk_params& P) {
    if (threadIdx.x != 0) return;
    int n = 0;
    for (int s = 0; s < P.n_stages; s++) {
        SR S = stage_at(P, s);
        if (S.kind == SK_ATTN) continue;
        const int nch = range_at(s).nch;
        for (int c = 0; c < nch && n < SK_MAX_CHUNKS; c++) l_cl()[1 + n++] = s | (c << 8) | (S.kind == SK_VOCAB ? SK_CL_VOCAB : 0);
    }
    l_cl()[0] = n;
}

// chunk list entry ci of step `step` -> the next chunk this workgroup computes (the word scores only from
// logits_from on); false when there is none
__device__ __forceinline__ bool next_chunk(const sk_params& P, int& step, int& ci, int& s, int& c) {
    const int n = l_cl()[0];
    int k = ci + 1;
    for (int guard = 0; guard < 2 * SK_MAX_CHUNKS + 4; guard++) {
        if (k >= n) {
            k = 0;
            if (++step >= P.n_steps || n == 0) return false;
        }
        const int e = l_cl()[1 + k];
        if ((e & SK_CL_VOCAB) && step < P.logits_from) { k = n; continue; }
        ci = k;
        s = e & 0xFF;
        c = (e >> 8) & 0xFF;
        return true;
    }
    return false;
}

template <int M>
__device__ __forceinline__ void issue(const sk_params& P, int b, int G, int s, int c, u32x4 (&w)[9]) {
    SR S = stage_at(P, s);
    const wg_range r = range_at(s);
    const int nu = min(r.cu, r.n - c * r.cu);
    const int g0 = (r.u0 + c * r.cu) * S.ug, ng = nu * S.ug, nb = S.W.nb;
    // every thread loads (threads past the chunk re-read its first pair), so the register set is written on every
    // path and the compiler's wait counting stays exact
    const int t = threadIdx.x < ng * nb ? threadIdx.x : 0;
    const int gi = t / nb, j = t - gi * nb, g = g0 + gi;
    const u32x4 GLB* codes = (const u32x4 GLB*)S.W.codes;
#pragma unroll
    for (int r8 = 0; r8 < 8; r8++) w[r8] = __builtin_nontemporal_load(codes + (size_t)(8 * g + r8) * nb + j);
    w[8] = __builtin_nontemporal_load((const u32x4 GLB*)S.W.scales + (size_t)g * nb + j);
}

// stage timestamps: per step, slot 0 = step start, then per stage 4 slots: prologue start, input arrived,
// chunks done, stage done
__device__ __forceinline__ void trace_at(const sk_params& P, int b, int k) {
    if (P.trace && threadIdx.x == 0 && k >= 0 && k < P.n_trace) ((long long GLB*)P.trace)[(size_t)b * P.n_trace + k] = wall_clock64();
}
__device__ __forceinline__ int tslot(const sk_params& P, int step, int s, int k) { return step * (1 + 4 * P.n_stages) + (s < 0 ? 0 : 1 + 4 * s + k); }

// ---------------------------------------------------------------- transposed x / y
__device__ __forceinline__ int xt_at(int i) { return (i & 31) * SK_XT_LD + (i >> 5); }

// gather destination in the transposed layout: index m * 2048 + i -> conversation m's value i
struct xt_dst {
    float LDS* base;
    __device__ __forceinline__ float LDS& operator[](int k) const { return base[(k >> 11) * SK_XT_M + xt_at(k & 2047)]; }
};

template <int NQ>
__device__ __forceinline__ float rms_scale_T(const float LDS* xt, float eps) { return rms_scale_xt<NQ, SK_XT_LD>(xt, eps); }

__device__ __forceinline__ float rms_T(const float LDS* xt, int n, float eps) {
    switch (n) {
        case 256: return rms_scale_T<2>(xt, eps);
        case 512: return rms_scale_T<4>(xt, eps);
        case 1024: return rms_scale_T<8>(xt, eps);
        default: return rms_scale_T<16>(xt, eps);
    }
}

// a quarter (values 4s .. 4s+3) of 32-value block j of conversation m cut to int8 (imi/core/vec.h:47-75) by the 8
// consecutive lanes s = 0..7 of the block: amax and the code sum are reduced across them (max and integer sums do
// not depend on order); lane s writes code word s; lane 0 the scale d and d * sum
__device__ __forceinline__ void cut_quad(const float (&h)[4], int m, int j, int s) {
    float amax = fmaxf(fmaxf(fabsf(h[0]), fabsf(h[1])), fmaxf(fabsf(h[2]), fabsf(h[3])));
    amax = fmaxf(amax, dppf<DPP_XOR1>(amax));
    amax = fmaxf(amax, dppf<DPP_XOR2>(amax));
    amax = fmaxf(amax, dppf<DPP_MIRROR8>(amax));
    const float d = amax / 127.0f;
    const float id = d != 0.0f ? 1.0f / d : 0.0f;
    int sum = 0;
    unsigned packed = 0;
#pragma unroll
    for (int k = 0; k < 4; k++) {
        const int c = (int)rintf(h[k] * id);
        sum += c;
        packed |= ((unsigned)c & 0xFFu) << (8 * k);
    }
    sum += dppi<DPP_XOR1>(sum);
    sum += dppi<DPP_XOR2>(sum);
    sum += dppi<DPP_MIRROR8>(sum);
    l_xq()[m * 2048 + 8 * j + s] = (int)packed;
    if (s == 0) {
        l_dx()[m * 256 + j] = d;
        l_s()[m * 256 + j] = d * (float)sum;
    }
}

// ---------------------------------------------------------------- prologues
// values 4s .. 4s+3 of block j of conversation m: h = x * sc * w_pre (imi_norm_mul, imi/core/vec.h:36-39), optionally
// written out (hid: the conversation's hidden row), then cut with the block's other 7 lanes (imi_q8::from,
// imi/core/tables.cpp:100-109)
__device__ __forceinline__ void norm_cut_quad(int m, int j, int s, float sc, const f32x4& w, float* hid, bool cut) {
    const float LDS* xc = l_x() + m * SK_XT_M + (4 * s) * SK_XT_LD + j;
    float h[4];
    h[0] = xc[0] * sc * w.x;
    h[1] = xc[SK_XT_LD] * sc * w.y;
    h[2] = xc[2 * SK_XT_LD] * sc * w.z;
    h[3] = xc[3 * SK_XT_LD] * sc * w.w;
    if (hid) *(f32x4 GLB*)(hid + 32 * j + 4 * s) = f32x4{h[0], h[1], h[2], h[3]};
    if (cut) cut_quad(h, m, j, s);
}

// x += norm(y) * w_post (imi_norm_mul_add, imi/core/vec.h:41-44); then h = norm(x) * w_pre and its cut. Threads
// are split by conversation (m = t / (512 / M)); every wave computes its conversation's norm scales itself (the
// same chain in every wave, so the same value), which saves two block barriers. The x update runs over 4-value
// row pieces of the transposed layout, the norm and cut over (block, quarter) pairs, E / 4 of each per conversation.
template <int M>
__device__ __forceinline__ bool pro_resid(const sk_params& P, SR S, unsigned tag, int par, float* hid0, float* hid1, bool cut, int tr) {
    constexpr int HALF = SK_THREADS / M;
    constexpr int QPT = 512 / HALF;   // pieces (and pairs) per thread at E = 2048
    const int E = P.E, t = threadIdx.x, m = t / HALF, tt = t - m * HALF, nqr = E / 128, npc = E / 4;
    // the post-norm weight is read before the wait, so it arrives with the input
    float wpost[QPT][4];
#pragma unroll
    for (int k = 0; k < QPT; k++) {
        const int q = tt + k * HALF;
        if (q < npc) {
            const int pr = q / nqr, t0 = 4 * (q - pr * nqr);
#pragma unroll
            for (int e = 0; e < 4; e++) wpost[k][e] = ((const float GLB*)S.w_post)[32 * (t0 + e) + pr];
        }
    }
    const bool ok = ll_gather(S.in + (size_t)par * 2 * S.n_in, S.n_in, E, M, tag, xt_dst{l_y()}, 2048, P);
    if (__syncthreads_or(!ok)) return false;
    trace_at(P, blockIdx.x, tr);
    const float sc1 = rms_T(l_y() + m * SK_XT_M, E, P.eps);
#pragma unroll
    for (int k = 0; k < QPT; k++) {
        const int q = tt + k * HALF;
        if (q < npc) {
            const int pr = q / nqr, t0 = 4 * (q - pr * nqr);
            const f32x4 y4 = *(const f32x4 LDS*)(l_y() + m * SK_XT_M + pr * SK_XT_LD + t0);
            f32x4 LDS* xp = (f32x4 LDS*)(l_x() + m * SK_XT_M + pr * SK_XT_LD + t0);
            f32x4 x4 = *xp;
            x4.x = fmaf(y4.x * sc1, wpost[k][0], x4.x);
            x4.y = fmaf(y4.y * sc1, wpost[k][1], x4.y);
            x4.z = fmaf(y4.z * sc1, wpost[k][2], x4.z);
            x4.w = fmaf(y4.w * sc1, wpost[k][3], x4.w);
            *xp = x4;
        }
    }
    f32x4 wpre[QPT];   // in flight during the second norm's chain
#pragma unroll
    for (int k = 0; k < QPT; k++) {
        const int q = tt + k * HALF;
        wpre[k] = q < npc ? *(const f32x4 GLB*)(S.w_pre + 4 * q) : f32x4{0, 0, 0, 0};   // block q / 8, quarter q % 8
    }
    __syncthreads();
    const float sc2 = rms_T(l_x() + m * SK_XT_M, E, P.eps);
#pragma unroll
    for (int k = 0; k < QPT; k++) {
        const int q = tt + k * HALF;
        if (q < npc) norm_cut_quad(m, q >> 3, q & 7, sc2, wpre[k], m == 0 ? hid0 : hid1, cut);
    }
    __syncthreads();
    return true;
}

template <int M>
__device__ __forceinline__ void pro_first(const sk_params& P, SR S) {
    constexpr int HALF = SK_THREADS / M;
    constexpr int QPT = 512 / HALF;
    const int E = P.E, t = threadIdx.x, m = t / HALF, tt = t - m * HALF, npc = E / 4;
    f32x4 wpre[QPT];
#pragma unroll
    for (int k = 0; k < QPT; k++) {
        const int q = tt + k * HALF;
        wpre[k] = q < npc ? *(const f32x4 GLB*)(S.w_pre + 4 * q) : f32x4{0, 0, 0, 0};
    }
    const float sc = rms_T(l_x() + m * SK_XT_M, E, P.eps);
#pragma unroll
    for (int k = 0; k < QPT; k++) {
        const int q = tt + k * HALF;
        if (q < npc) norm_cut_quad(m, q >> 3, q & 7, sc, wpre[k], nullptr, true);
    }
    __syncthreads();
}

// the previous table's float output, cut to int8 per 32 (imi/core/vec.h:47-75)
template <int M>
__device__ __forceinline__ bool pro_cut(const sk_params& P, SR S, unsigned tag, int par, int tr) {
    const int t = threadIdx.x;
    if (S.cut_in) {   // already cut by the producer: 10 records per block (8 code words, d, d * sum)
        const int n = S.n_in;
        const bool ok = ll_gather(S.in + (size_t)par * 2 * S.n_in, S.n_in, n, M, tag, l_stg(), 8192, P);
        if (__syncthreads_or(!ok)) return false;
        trace_at(P, blockIdx.x, tr);
#pragma unroll
        for (int m = 0; m < M; m++)
            for (int k = t; k < n; k += SK_THREADS) {
                const int blk = k / 10, w = k - blk * 10;
                const float v = l_stg()[m * 8192 + k];
                if (w < 8) l_xq()[m * 2048 + 8 * blk + w] = __float_as_int(v);
                else if (w == 8) l_dx()[m * 256 + blk] = v;
                else l_s()[m * 256 + blk] = v;
            }
        __syncthreads();
        return true;
    }
    const int K = S.n_in;
    const bool ok = ll_gather(S.in + (size_t)par * 2 * S.n_in, S.n_in, K, M, tag, l_stg(), 8192, P);
    if (__syncthreads_or(!ok)) return false;
    trace_at(P, blockIdx.x, tr);
    const int npc = K / 4;   // (block, quarter) pairs per conversation; 8 consecutive lanes per block
    for (int k = t; k < M * npc; k += SK_THREADS) {
        const int m = k / npc, q = k - m * npc;
        const f32x4 a = *(const f32x4 LDS*)(l_stg() + m * 8192 + 4 * q);
        const float h[4] = {a.x, a.y, a.z, a.w};
        cut_quad(h, m, q >> 3, q & 7);
    }
    __syncthreads();
    return true;
}

// ---------------------------------------------------------------- GEMV chunk
// phase 1: thread = (group gi, block j); exact integer dots of the 8 rows against each input's cut block; the
// chain operands float(isum) and d * dx to LDS row-major ([input][row][block], rows padded to st so 16-byte reads
// by the lanes of a wave are conflict free), with the rows' scales d beside them ([row][block])
template <int M>
__device__ __forceinline__ void phase1(const u32x4 (&w)[9], int ng, int nb, int rows) {
    const int t = threadIdx.x;
    if (t < ng * nb) {
        const int gi = t / nb, j = t - gi * nb, st = sk_row_stride(nb);
        float d[8];
        const unsigned sw[4] = {w[8].x, w[8].y, w[8].z, w[8].w};
#pragma unroll
        for (int r = 0; r < 8; r++) d[r] = h2f((uint16_t)((r & 1) ? (sw[r >> 1] >> 16) : (sw[r >> 1] & 0xFFFFu)));
#pragma unroll
        for (int m = 0; m < M; m++) {
            int xq[8];
            const u32x4 LDS* xs = (const u32x4 LDS*)(l_xq() + m * 2048 + 8 * j);
            const u32x4 a = xs[0], c = xs[1];
            xq[0] = (int)a.x; xq[1] = (int)a.y; xq[2] = (int)a.z; xq[3] = (int)a.w;
            xq[4] = (int)c.x; xq[5] = (int)c.y; xq[6] = (int)c.z; xq[7] = (int)c.w;
            const float dx = l_dx()[m * 256 + j];
            float LDS* op = l_pq() + (m * rows + 8 * gi) * st + j;              // float(isum)
            float LDS* oq = l_pq() + ((M + m) * rows + 8 * gi) * st + j;        // d * dx
#pragma unroll
            for (int r = 0; r < 8; r++) {
                op[r * st] = (float)q4_block_dot(w[r], xq);
                oq[r * st] = d[r] * dx;
            }
        }
        float LDS* dd = l_dd() + (8 * gi) * st + j;
#pragma unroll
        for (int r = 0; r < 8; r++) dd[r * st] = d[r];
    }
}

// conv taps and memory of this thread's channel, loaded before the chunk's prefetch is issued (a global load in
// the epilogue would wait for that prefetch: loads complete in order)
struct conv_pre {
    float w[SK_CONV_MAX + 1], st[SK_CONV_MAX];
};

template <int M>
__device__ __forceinline__ void conv_load(const sk_params& P, SR S, int g0, int C, int rows, conv_pre& cp) {
    const int t = threadIdx.x;
    if (S.epi != SKE_CONV || t >= C) return;
    const int m = t / rows, rr = t - m * rows, k = rr % 24;
    if (k >= 8) return;
    const int E = P.E, dc = P.d_conv, e = 8 * (g0 / 3 + rr / 24) + k;
    const float GLB* st = (const float GLB*)((m == 0 ? P.cv[0].conv : P.cv[M - 1].conv) + (size_t)S.conv_layer * dc * E);
    const float GLB* cw = (const float GLB*)S.conv_w;
#pragma unroll
    for (int q = 0; q <= SK_CONV_MAX; q++)
        if (q <= dc) cp.w[q] = cw[(size_t)q * E + e];
#pragma unroll
    for (int q = 0; q < SK_CONV_MAX; q++)
        if (q < dc) cp.st[q] = st[(size_t)q * E + e];
}

template <int M>
__device__ __forceinline__ void phase2_epilogue(const sk_params& P, SR S, int g0, int C, int rows, unsigned tag, int par,
                                                float (&bv)[M], int (&bi)[M], const conv_pre& cp) {
    const int t = threadIdx.x, nb = S.W.nb;
    // imi's two chains per (input m, row) over the blocks in order (imi/core/tables.cpp:127-143): acc =
    // fma(float(isum), d * dx, acc) and cor = fma(d, s, cor), each wave issuing one FMA per step; out = fma(-8, cor,
    // acc). Chain c's acc runs on lane 128 (c / 64) + c % 64 and its cor 64 lanes further, so the two waves of a
    // 128-lane pair sit on different SIMDs and the two chains of a row do not share one SIMD's issue slots. Operands
    // come 4 blocks per 16-byte LDS read, with the reads of the next 24 blocks in flight while the chain runs.
    const int cw = t >> 6, cc = 64 * (cw >> 1) + (t & 63);
    const bool acc_lane = (cw & 1) == 0 && cc < C, cor_lane = (cw & 1) == 1 && cc < C;
    float chain = 0.0f;
    if (acc_lane || cor_lane) {
        const int c = cc, m = c / rows, r = c - m * rows, st = sk_row_stride(nb);
        const f32x4 LDS* ap = (const f32x4 LDS*)(acc_lane ? l_pq() + (m * rows + r) * st : l_dd() + r * st);
        const f32x4 LDS* bp = (const f32x4 LDS*)(acc_lane ? l_pq() + ((M + m) * rows + r) * st : l_s() + m * 256);
        const int n4 = nb / 4;
#define SK_STEP4(A4, B4)                                                                              \
        chain = fmaf(A4.x, B4.x, chain); chain = fmaf(A4.y, B4.y, chain);                             \
        chain = fmaf(A4.z, B4.z, chain); chain = fmaf(A4.w, B4.w, chain);
        if ((n4 & 15) == 0) {   // per 64 blocks: the reads of the next 7 quads (28 blocks) in flight ahead
            for (int q0 = 0; q0 < n4; q0 += 16) {
                f32x4 qa[16], qb[16];
#pragma unroll
                for (int k = 0; k < 6; k++) { qa[k] = ap[q0 + k]; qb[k] = bp[q0 + k]; }
#pragma unroll
                for (int k = 0; k < 16; k++) {
                    if (k + 6 < 16) { qa[k + 6] = ap[q0 + k + 6]; qb[k + 6] = bp[q0 + k + 6]; }
                    __builtin_amdgcn_sched_barrier(0);   // keep the reads ahead of the chain
                    SK_STEP4(qa[k], qb[k])
                }
            }
        } else {
            const float LDS* as = (const float LDS*)ap;
            const float LDS* bs = (const float LDS*)bp;
            for (int j = 0; j < nb; j++) chain = fmaf(as[j], bs[j], chain);
        }
#undef SK_STEP4
        if (cor_lane) l_cor()[c] = chain;
    }
    __syncthreads();
    if (acc_lane) l_out()[cc] = fmaf(-8.0f, l_cor()[cc], chain);
    __syncthreads();
    const float outv = t < C ? l_out()[t] : 0.0f;
    if (t >= C) return;
    const int m = t / rows, rr = t - m * rows;
    u64* out = S.out ? S.out + (size_t)(par * 2 + m) * S.n_out : nullptr;
    if (S.epi == SKE_STORE) {
        ll_put(out + 8 * g0 + rr, outv, tag);
    } else if (S.epi == SKE_SWIGLU) {   // (gate group, up group) of 8 FFN channels (imi/core/seoul.cpp:380-394)
        const int k = rr & 15;
        if (k < 8) {
            const float a = silu(outv) * l_out()[t + 8];
            // cut_out: the chunk's channels go to LDS and are cut and published per 32 after the block barrier
            if (S.cut_out) l_cor()[m * (rows / 2) + 8 * (rr / 16) + k] = a;
            else ll_put(out + 8 * (g0 / 2 + rr / 16) + k, a, tag);
        }
    } else if (S.epi == SKE_CONV) {     // (b, c, x) groups of 8 channels (imi/core/seoul.cpp:407-423)
        const int k = rr % 24;
        if (k < 8) {
            const int E = P.E, dc = P.d_conv, e = 8 * (g0 / 3 + rr / 24) + k;
            const float cc = l_out()[t + 8], xx = l_out()[t + 16];
            float GLB* st = (float GLB*)((m == 0 ? P.cv[0].conv : P.cv[M - 1].conv) + (size_t)S.conv_layer * dc * E);
            const float bx = outv * xx;
            float wdc = cp.w[0];
#pragma unroll
            for (int q = 1; q <= SK_CONV_MAX; q++)
                if (q == dc) wdc = cp.w[q];
            float uu = outv * xx * wdc;
#pragma unroll
            for (int q = 0; q < SK_CONV_MAX; q++)
                if (q < dc) uu = fmaf(cp.st[q], cp.w[q], uu);
            uu *= cc;
#pragma unroll
            for (int q = 0; q + 1 < SK_CONV_MAX; q++)
                if (q + 1 < dc) st[(size_t)q * E + e] = cp.st[q + 1];
            st[(size_t)(dc - 1) * E + e] = bx;
            ll_put(out + e, uu, tag);
        }
    } else {   // SKE_LOGITS
        const int row = 8 * g0 + rr;
        float* lg = m == 0 ? P.cv[0].logits : P.cv[M - 1].logits;
        if (lg) ((float GLB*)lg)[row] = outv;
#pragma unroll
        for (int mm = 0; mm < M; mm++)
            if (mm == m && (outv > bv[mm] || (outv == bv[mm] && row < bi[mm]))) { bv[mm] = outv; bi[mm] = row; }
    }
}

// first index of the maximum over the block: each thread offers (v, i); every thread gets the winner
__device__ __forceinline__ void block_argmax(float v, int i, float* out_v, int* out_i) {
    const int t = threadIdx.x, lane = t & 63, wv = t >> 6;
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
        const float ov = __shfl_xor(v, o);
        const int oi = __shfl_xor(i, o);
        if (ov > v || (ov == v && oi < i)) { v = ov; i = oi; }
    }
    __syncthreads();
    if (lane == 0) { l_redv()[wv] = v; l_redi()[wv] = i; }
    __syncthreads();
    v = l_redv()[0];
    i = l_redi()[0];
    for (int k = 1; k < SK_THREADS / 64; k++) {
        const float ov = l_redv()[k];
        const int oi = l_redi()[k];
        if (ov > v || (ov == v && oi < i)) { v = ov; i = oi; }
    }
    *out_v = v;
    *out_i = i;
    __syncthreads();
}

// the word chosen by a step: first index of the maximum over the workgroups' partials of conversation m
__device__ __forceinline__ bool reduce_partials(const sk_params& P, unsigned tag, int G, int m, int* best) {
    const int par = tag & 1, t = threadIdx.x;
    float v = -INFINITY;
    int i = 0x7fffffff;
    bool ok = true;
    if (t < G) {
        const u64* pv = P.part + (((size_t)par * 2 + m) * 2) * G;
        u64 rv = ll_load(pv + t), ri = ll_load(pv + G + t);
        if ((unsigned)(rv >> 32) != tag) { float x; ok = ll_wait(pv + t, tag, &x, P); rv = __float_as_uint(x); }
        if (ok && (unsigned)(ri >> 32) != tag) { float x; ok = ll_wait(pv + G + t, tag, &x, P); ri = __float_as_uint(x); }
        v = __uint_as_float((unsigned)rv);
        i = (int)(unsigned)ri;
    }
    if (__syncthreads_or(!ok)) return false;
    float bvv;
    block_argmax(v, i, &bvv, best);
    return true;
}

// ---------------------------------------------------------------- attention (imi/core/seoul.cpp:424-461)
// workgroup (kv head g, conversation m): k = rope(norm(k) * k_norm), v to the fp16 cache at pos; per query head of
// the group: q = rope(norm(q) * q_norm), scores = dot_h(q, K_t) / sqrt(D), softmax with the max subtracted, glibc's
// expf and a double sum in position order, o = sum_t fma(e_t * inv, V_t, o) in order, times the sigmoid head gate
template <int D>
__device__ __forceinline__ bool attention(const sk_params& P, SR S, int g, int m, int pos, unsigned tag, int par) {
    constexpr int half = D / 2;
    const int t = threadIdx.x, lane = t & 63, wv = t >> 6;
    const int grp = P.n_head / P.n_kv, Hq = P.n_head * D, kvd = P.n_kv * D, n_ctx = P.n_ctx;
    const int s0 = (S.swa && P.n_swa > 0) ? max(0, pos - P.n_swa + 1) : 0, nk = pos - s0 + 1;
    uint16_t GLB* kc = (uint16_t GLB*)(P.cv[m].kc + ((size_t)S.layer_ai * P.n_kv + g) * n_ctx * D);
    uint16_t GLB* vc = (uint16_t GLB*)(P.cv[m].vc + ((size_t)S.layer_ai * P.n_kv + g) * n_ctx * D);
    float LDS* row = l_att();                    // [grp*D | k D | v D | gates grp]
    float LDS* q_s = row + 512;                  // [grp][D]
    float LDS* scratch = q_s + 8 * D;            // [9][D]
    float LDS* inv_s = scratch + 9 * D;          // [8]
    float LDS* sc = inv_s + 8;                   // [grp][n_ctx]
    const int n_need = grp * D + 2 * D + grp;
    bool ok = true;
    if (t < n_need) {
        int idx;
        if (t < grp * D) idx = g * grp * D + t;
        else if (t < grp * D + D) idx = Hq + g * D + (t - grp * D);
        else if (t < grp * D + 2 * D) idx = Hq + kvd + g * D + (t - grp * D - D);
        else idx = Hq + 2 * kvd + g * grp + (t - grp * D - 2 * D);
        float v;
        ok = ll_wait(S.in + (size_t)(par * 2 + m) * S.n_in + idx, tag, &v, P);
        row[t] = v;
    }
    if (__syncthreads_or(!ok)) return false;
    const float GLB* cs = (const float GLB*)S.rope_cs + (size_t)pos * D;   // (cos, sin) pairs
    // norm + NEOX rope of one head vector, one wave (imi/core/seoul.cpp:19-28; angles from the host's table)
    for (int hh = wv; hh <= grp; hh += SK_THREADS / 64) {
        const bool is_k = hh == grp;
        const float LDS* src = is_k ? row + grp * D : row + hh * D;
        const float GLB* w = (const float GLB*)(is_k ? S.k_norm : S.q_norm);
        float LDS* dst = is_k ? scratch + 8 * D : q_s + hh * D;
        float LDS* st = scratch + wv * D;
        const float x = lane < D ? src[lane] : 0.0f;
        if (lane < D) st[lane] = x;
        __builtin_amdgcn_wave_barrier();
        const float s = rms_scale_wave((const float LDS*)st, D, P.eps);
        const float n = lane < D ? x * s * w[lane] : 0.0f;
        const float other = __shfl(n, lane < half ? lane + half : lane - half);
        if (lane < D) {
            const int ci = lane < half ? lane : lane - half;
            const float co = cs[2 * ci], si = cs[2 * ci + 1];
            const float r = lane < half ? fmaf(n, co, -(other * si)) : fmaf(other, si, n * co);
            dst[lane] = r;
            if (is_k) {
                kc[(size_t)pos * D + lane] = f2h(r);
                vc[(size_t)pos * D + lane] = f2h(row[grp * D + D + lane]);
            }
        }
        __builtin_amdgcn_wave_barrier();
    }
    __syncthreads();
    const float scale = 1.0f / sqrtf((float)D);
    for (int q = t; q < nk; q += SK_THREADS) {
        const u32x4 GLB* kt = (const u32x4 GLB*)(kc + (size_t)(s0 + q) * D);
        unsigned kw[D / 2];   // the key row as fp16 pairs, converted per use (keeps the registers low)
#pragma unroll
        for (int i0 = 0; i0 < D / 8; i0++) {
            const u32x4 w4 = kt[i0];
            kw[4 * i0] = w4.x; kw[4 * i0 + 1] = w4.y; kw[4 * i0 + 2] = w4.z; kw[4 * i0 + 3] = w4.w;
        }
        for (int hh = 0; hh < grp; hh++) {
            // dot_h (imi/core/seoul.cpp:29-39): 8 FMA chains over columns i % 8, then the 8-lane horizontal sum
            const float LDS* qh = q_s + hh * D;
            float a[8];
#pragma unroll
            for (int l = 0; l < 8; l++) a[l] = 0.0f;
#pragma unroll
            for (int i = 0; i < D; i += 8)
#pragma unroll
                for (int l = 0; l < 8; l++) a[l] = fmaf(qh[i + l], h2f((uint16_t)(kw[(i + l) >> 1] >> (16 * (l & 1)))), a[l]);
            sc[hh * n_ctx + q] = (((a[0] + a[4]) + (a[2] + a[6])) + ((a[1] + a[5]) + (a[3] + a[7]))) * scale;
        }
    }
    __syncthreads();
    for (int hh = wv; hh < grp; hh += SK_THREADS / 64) {
        float LDS* s = sc + hh * n_ctx;
        float mx = -INFINITY;
        for (int q = lane; q < nk; q += 64) mx = fmaxf(mx, s[q]);
        mx = wave_max(mx);
        for (int q = lane; q < nk; q += 64) s[q] = expf_glibc(s[q] - mx);
        __builtin_amdgcn_wave_barrier();
        if (lane == 0) {
            double sum = 0.0;
            int q = 0;
            for (; q + 8 <= nk; q += 8) {
                float v[8];
#pragma unroll
                for (int u = 0; u < 8; u++) v[u] = s[q + u];
#pragma unroll
                for (int u = 0; u < 8; u++) sum += (double)v[u];
            }
            for (; q < nk; q++) sum += (double)s[q];
            inv_s[hh] = (float)(1.0 / sum);
        }
    }
    __syncthreads();
    // o = sum_t fma(e_t * inv, V_t, o): the window's value rows pass through LDS in tiles (one coalesced load per
    // tile instead of a dependent global load per position), the chain itself stays in position order
    float LDS* vt = sc + grp * n_ctx;
    const int tv = min(256, ((SK_ATTN_BYTES / 4 - (int)(vt - row)) / D) & ~7);
    const int k = t;                               // thread = (query head hh, dimension i); grp * D <= 512
    const int hh = k / D, i = k - hh * D;
    const bool on = k < grp * D;
    const float inv = on ? inv_s[hh] : 0.0f;
    const float LDS* sh = sc + (on ? hh : 0) * n_ctx;
    float o = 0.0f;
    for (int q0 = 0; q0 < nk; q0 += tv) {
        const int nt = min(tv, nk - q0);
        const u32x4 GLB* src = (const u32x4 GLB*)(vc + (size_t)(s0 + q0) * D);
        for (int e = t; e < nt * D / 8; e += SK_THREADS) {
            const u32x4 w4 = src[e];
            const unsigned hw[4] = {w4.x, w4.y, w4.z, w4.w};
            float LDS* dst = vt + 8 * e;
#pragma unroll
            for (int h = 0; h < 8; h++) dst[h] = h2f((uint16_t)(hw[h >> 1] >> (16 * (h & 1))));
        }
        __syncthreads();
        if (on) {
            int q = 0;
            for (; q + 8 <= nt; q += 8) {
                float e[8], v[8];
#pragma unroll
                for (int u = 0; u < 8; u++) { e[u] = sh[q0 + q + u]; v[u] = vt[(q + u) * D + i]; }
#pragma unroll
                for (int u = 0; u < 8; u++) o = fmaf(e[u] * inv, v[u], o);
            }
            for (; q < nt; q++) o = fmaf(sh[q0 + q] * inv, vt[q * D + i], o);
        }
        __syncthreads();
    }
    if (on) {
        const float gate = 1.0f / (1.0f + expf_glibc(-row[grp * D + 2 * D + hh]));
        u64* out = S.out + (size_t)(par * 2 + m) * S.n_out;
        ll_put(out + (g * grp + hh) * D + i, o * gate, tag);
    }
    __syncthreads();
    return true;
}



// ---------------------------------------------------------------- the walk over one workgroup's work
// Per workgroup, a launch is a sequence of chunks with other work in between (embedding, prologues, attention,
// the end of the word scores). `events` runs that work up to the next chunk; `chunk` issues the loads of the
// chunk after it into the other register set and computes this one. The kernel alternates the two sets
// explicitly, so neither is copied and the prefetch stays in flight.
struct walk_state {
    int step, s, c, nch;
    bool embedded, pro_done;
    int ci;   // chunk list index of the next chunk computed
};

__device__ __forceinline__ void next_stage(const sk_params& P, walk_state& W) {
    W.s++;
    W.c = 0;
    W.pro_done = false;
    if (W.s == P.n_stages) {
        W.s = 0;
        W.step++;
        W.embedded = false;
    }
}

// the step's input rows (imi/core/seoul.cpp:363-364): word-table row of the token, or the given vector
template <int M>
__device__ __forceinline__ bool embed(const sk_params& P, walk_state& W, int b, int G) {
    const unsigned tag = P.epoch0 + (unsigned)W.step;
    const int t = threadIdx.x;
    trace_at(P, b, tslot(P, W.step, -1, 0));
    int tok0 = 0, tok1 = 0;
    if (P.greedy && W.step > 0) {
        if (b == 0) {
            tok0 = l_misci()[0];
            tok1 = l_misci()[1];
        } else {
            if (!reduce_partials(P, tag - 1, G, 0, &tok0)) return false;
            if (M == 2 && !reduce_partials(P, tag - 1, G, 1, &tok1)) return false;
        }
    } else if (P.greedy) {
        tok0 = P.cv[0].first_token;
        tok1 = P.cv[M - 1].first_token;
    } else {
        tok0 = ((const int GLB*)P.cv[0].tokens)[W.step];
        tok1 = ((const int GLB*)P.cv[M - 1].tokens)[W.step];
    }
    if (tok0 >= P.V) tok0 = 0;   // no maximum (all scores NaN): row 0, never out of the table
    if (tok1 >= P.V) tok1 = 0;
    const int nbE = P.E / 32;
    if (t < M * nbE) {
        const int m = t / nbE, j = t - m * nbE;
        const int tok = m == 0 ? tok0 : tok1;
        float v[32];
        if (tok >= 0) {
            const u32x4 cw = ((const u32x4 GLB*)P.vocab.codes)[(size_t)tok * P.vocab.nb + j];
            const uint16_t dh = ((const uint16_t GLB*)P.vocab.scales)[((size_t)(tok >> 3) * P.vocab.nb + j) * 8 + (tok & 7)];
            const float d = h2f(dh);
            const unsigned w4[4] = {cw.x, cw.y, cw.z, cw.w};
#pragma unroll
            for (int i = 0; i < 16; i++) {
                const unsigned byte = (w4[i >> 2] >> (8 * (i & 3))) & 0xFFu;
                v[i] = (float)((int)(byte & 15u) - 8) * d;
                v[16 + i] = (float)((int)(byte >> 4) - 8) * d;
            }
        } else {
            const float* eb = m == 0 ? P.cv[0].embd : P.cv[M - 1].embd;
            const f32x4 GLB* e = (const f32x4 GLB*)(eb + (size_t)W.step * P.E + 32 * j);
#pragma unroll
            for (int q = 0; q < 8; q++) {
                const f32x4 a = e[q];
                v[4 * q] = a.x; v[4 * q + 1] = a.y; v[4 * q + 2] = a.z; v[4 * q + 3] = a.w;
            }
        }
        float LDS* x = l_x() + m * SK_XT_M + j;   // values 32 j + i at row i, column j
#pragma unroll
        for (int i = 0; i < 32; i++) x[i * SK_XT_LD] = v[i];
    }
    __syncthreads();
    return true;
}

// runs everything up to the next chunk; false when the launch is done (or a wait failed)
template <int M>
__device__ __forceinline__ bool events(const sk_params& P, walk_state& W, int b, int G, float (&bv)[M], int (&bi)[M]) {
    for (;;) {
        if (W.step >= P.n_steps) return false;
        const unsigned tag = P.epoch0 + (unsigned)W.step;
        const int par = tag & 1;
        if (!W.embedded) {
            if (!embed<M>(P, W, b, G)) return false;
            W.embedded = true;
#pragma unroll
            for (int m = 0; m < M; m++) { bv[m] = -INFINITY; bi[m] = 0x7fffffff; }
        }
        SR S = stage_at(P, W.s);
        if (!W.pro_done) {
            trace_at(P, b, tslot(P, W.step, W.s, 0));
            if (S.kind == SK_ATTN) {
                if (b < P.n_kv * M) {
                    const int g = b % P.n_kv, m = b / P.n_kv;
                    const int pos = P.cv[m].pos + W.step;
                    const bool ok = P.D == 64 ? attention<64>(P, S, g, m, pos, tag, par) : attention<32>(P, S, g, m, pos, tag, par);
                    if (!ok) return false;
                }
                trace_at(P, b, tslot(P, W.step, W.s, 3));
                next_stage(P, W);
                continue;
            }
            float* hid0 = nullptr;
            float* hid1 = nullptr;
            if (S.kind == SK_VOCAB && b == 0) {
                if (P.cv[0].hidden) hid0 = P.cv[0].hidden + (size_t)W.step * P.cv[0].hidden_stride;
                if (M == 2 && P.cv[1].hidden) hid1 = P.cv[1].hidden + (size_t)W.step * P.cv[1].hidden_stride;
            }
            if (S.kind == SK_VOCAB && W.step < P.logits_from) {   // no word scores: the final norm only
                if (b == 0 && !pro_resid<M>(P, S, tag, par, hid0, hid1, false, tslot(P, W.step, W.s, 1))) return false;
                trace_at(P, b, tslot(P, W.step, W.s, 3));
                next_stage(P, W);
                continue;
            }
            W.nch = range_at(W.s).nch;
            bool ok = true;
            if (S.pro == SKP_RESID) ok = pro_resid<M>(P, S, tag, par, hid0, hid1, true, tslot(P, W.step, W.s, 1));
            else if (S.pro == SKP_FIRST) pro_first<M>(P, S);
            else if (W.nch > 0) ok = pro_cut<M>(P, S, tag, par, tslot(P, W.step, W.s, 1));
            if (!ok) return false;
            W.pro_done = true;
        }
        if (W.c < W.nch) return true;
        // the stage is done
        trace_at(P, b, tslot(P, W.step, W.s, 2));
        if (S.epi == SKE_LOGITS) {
#pragma unroll
            for (int m = 0; m < M; m++) {
                float v;
                int i;
                block_argmax(bv[m], bi[m], &v, &i);
                if (threadIdx.x == 0) {
                    u64* pv = P.part + (((size_t)par * 2 + m) * 2) * G;
                    ll_put(pv + b, v, tag);
                    ll_put(pv + G + b, __int_as_float(i), tag);
                }
            }
            if (b == 0) {
#pragma unroll
                for (int m = 0; m < M; m++) {
                    int best = 0;
                    if (!reduce_partials(P, tag, G, m, &best)) return false;
                    if (threadIdx.x == 0) {
                        l_misci()[m] = best;
                        int32_t* ids = m == 0 ? P.cv[0].ids : P.cv[M - 1].ids;
                        if (ids) ((int GLB*)ids)[W.step] = best;
                    }
                }
                __syncthreads();
            }
        }
        trace_at(P, b, tslot(P, W.step, W.s, 3));
        next_stage(P, W);
    }
}

// chunk (step, s, c): issue the next chunk's loads into nxt, compute this one from cur
template <int M>
__device__ __forceinline__ void chunk(const sk_params& P, walk_state& W, int b, int G, float (&bv)[M], int (&bi)[M],
                                      const u32x4 (&cur)[9], u32x4 (&nxt)[9]) {
    const unsigned tag = P.epoch0 + (unsigned)W.step;
    const int par = tag & 1;
    SR S = stage_at(P, W.s);
    const wg_range r = range_at(W.s);
    const int nu = min(r.cu, r.n - W.c * r.cu);
    const int g0 = (r.u0 + W.c * r.cu) * S.ug, ng = nu * S.ug, rows = 8 * ng, C = M * rows;
    conv_pre cp;
    conv_load<M>(P, S, g0, C, rows, cp);
    // the next chunk's loads go out after this chunk's results are published: the issue cost is off the path to
    // the publish, and the stream overlaps the wait for the next stage's input
    int qs = W.step, qci = W.ci, qss = W.s, qc = W.c;
    if (!next_chunk(P, qs, qci, qss, qc)) { qss = W.s; qc = W.c; }   // the last chunk: a harmless re-read
    W.ci = qci;
    phase1<M>(cur, ng, S.W.nb, rows);
    __syncthreads();
    phase2_epilogue<M>(P, S, g0, C, rows, tag, par, bv, bi, cp);
    if (S.cut_out) {   // the chunk's rows / 2 FFN channels of each conversation, cut per 32 (imi/core/vec.h:47-75)
        __syncthreads();
        const int nblk = rows / 64;   // 32 channels = 4 units = 64 rows
        if (threadIdx.x < M * nblk) {
            const int m = threadIdx.x / nblk, k = threadIdx.x - m * nblk;
            float v[32];
            const float LDS* a = l_cor() + m * (rows / 2) + 32 * k;
#pragma unroll
            for (int i = 0; i < 32; i++) v[i] = a[i];
            int q8[8], sum;
            const float d = cut32(v, q8, &sum, false);
            u64* o = S.out + (size_t)(par * 2 + m) * S.n_out + (size_t)(g0 / 8 + k) * 10;
#pragma unroll
            for (int w = 0; w < 8; w++) ll_put(o + w, __int_as_float(q8[w]), tag);
            ll_put(o + 8, d, tag);
            ll_put(o + 9, d * (float)sum, tag);
        }
    }
    issue<M>(P, b, G, qss, qc, nxt);
    __syncthreads();
    W.c++;
}

}  // namespace

// ---------------------------------------------------------------- the kernel
template <int M>
__global__ __launch_bounds__(SK_THREADS, 1) void k_step(sk_params P) {
    const int b = blockIdx.x, G = gridDim.x;
    walk_state W{0, 0, 0, 0, false, false, -1};
    float bv[M];
    int bi[M];
#pragma unroll
    for (int m = 0; m < M; m++) { bv[m] = -INFINITY; bi[m] = 0x7fffffff; }
    for (int k = threadIdx.x; k < P.n_stages; k += SK_THREADS) {
        const wg_range r = compute_range<M>(stage_at(P, k), b, G);
        l_rng()[k] = i32x4{r.u0, r.n, r.cu, r.nch};
    }
    __syncthreads();
    build_chunk_list<M>(P);
    __syncthreads();
    u32x4 wa[9], wb[9];
    {
        int st = 0, s = 0, c = -1;
        if (next_chunk(P, st, W.ci, s, c)) issue<M>(P, b, G, s, c, wa);
    }
    for (;;) {
        if (!events<M>(P, W, b, G, bv, bi)) break;
        chunk<M>(P, W, b, G, bv, bi, wa, wb);
        if (!events<M>(P, W, b, G, bv, bi)) break;
        chunk<M>(P, W, b, G, bv, bi, wb, wa);
    }
}

hipError_t launch_step_kernel(int M, const sk_params& p, int grid, hipStream_t s) {
    const void* fn = M == 2 ? (const void*)k_step<2> : (const void*)k_step<1>;
    hipError_t e = hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, SK_LDS_BYTES);
    if (e != hipSuccess) return e;
    sk_params copy = p;
    void* args[] = {&copy};
    return hipLaunchCooperativeKernel(fn, dim3(grid), dim3(SK_THREADS), args, SK_LDS_BYTES, s);
}

hipError_t step_kernel_occupancy(int M, int* blocks_per_cu) {
    const void* fn = M == 2 ? (const void*)k_step<2> : (const void*)k_step<1>;
    hipError_t e = hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, SK_LDS_BYTES);
    if (e != hipSuccess) return e;
    return hipOccupancyMaxActiveBlocksPerMultiprocessor(blocks_per_cu, fn, SK_THREADS, SK_LDS_BYTES);
}

}  // namespace sh
