// ORACLE — test infrastructure only. Nothing under nunchi_amd/ includes, links or calls this.
//
// A from-scratch CPU restatement of imi's arithmetic for the brain step (the reference's AVX2 engine,
// imi/core/{vec.h,tables.cpp,seoul.cpp}, imi/kernels/q4x8.cpp, imi/core/voice.cpp). It is the checker the HIP path
// is compared with, and, timed on the host cores, the CPU baseline ("imi-cpu").
//
// Every function cites the reference file:line it follows. Where the reference fixes an op order (AVX2 lane
// layouts, FMA chains), the restatement keeps it, because that order is what parity is measured against.
// Parity pins for each function live in tests/ (closed forms, brute force, invariants); see the header of
// tests/test_oracle_*.py.
#pragma once
#include <immintrin.h>

#include <atomic>
#include <cstddef>
#include <cstdint>
#include <functional>
#include <string>
#include <thread>
#include <vector>

namespace orc {

// ---------------------------------------------------------------- thread team (shape of imi/core/team.h)
struct team {
    int n = 1;
    std::vector<std::thread> th;
    const std::function<void(int)>* job = nullptr;
    alignas(64) std::atomic<int> gen{0};
    alignas(64) std::atomic<int> done{0};
    alignas(64) std::atomic<int> arrived{0};
    alignas(64) std::atomic<int> phase{0};
    std::atomic<bool> quit{false};
    template <class F> static void wait_until(F ok) {
        for (int spins = 0; !ok();) { if (spins < 20000) { _mm_pause(); spins++; } else std::this_thread::yield(); }
    }
    void start(int nt) {
        n = nt < 1 ? 1 : nt;
        for (int t = 1; t < n; t++)
            th.emplace_back([this, t] {
                int seen = 0;
                for (;;) {
                    wait_until([&] { return gen.load(std::memory_order_acquire) != seen; });
                    seen = gen.load(std::memory_order_acquire);
                    if (quit.load()) return;
                    (*job)(t);
                    done.fetch_add(1, std::memory_order_acq_rel);
                }
            });
    }
    void run(const std::function<void(int)>& f) {
        job = &f;
        done.store(0, std::memory_order_relaxed);
        gen.fetch_add(1, std::memory_order_release);
        f(0);
        wait_until([&] { return done.load(std::memory_order_acquire) == n - 1; });
    }
    void sync() {   // spinning barrier (imi/core/team.h:39-48)
        if (n == 1) return;
        const int p = phase.load(std::memory_order_acquire);
        if (arrived.fetch_add(1, std::memory_order_acq_rel) == n - 1) {
            arrived.store(0, std::memory_order_relaxed);
            phase.store(p + 1, std::memory_order_release);
        } else {
            wait_until([&] { return phase.load(std::memory_order_acquire) != p; });
        }
    }
    ~team() {
        quit.store(true);
        gen.fetch_add(1, std::memory_order_release);
        for (auto& t : th) t.join();
    }
};

// ---- fp16 <-> fp32 (imi/core/tables.cpp:20-38) ----
float    h2f(uint16_t h);          // exact, bit construction as imi_h2f
uint16_t f2h(float f);             // round to nearest even (F16C _cvtss_sh(f, 0))

// ---- GGUF (minimal reader, own code; format: GGUF v3) ----
enum gtype : int { T_F32 = 0, T_F16 = 1, T_Q4_0 = 2, T_Q4_1 = 3, T_Q8_0 = 8, T_Q6_K = 14 };
struct gtensor {
    std::string name;
    int type = 0, n_dims = 0;
    int64_t ne[4] = {1, 1, 1, 1};
    size_t offset = 0, nbytes = 0, row_bytes = 0;
    const uint8_t* data = nullptr;
};
struct gfile {
    std::vector<gtensor> tensors;
    struct kv { std::string key; int type; int64_t i; double f; std::vector<int64_t> arr; };
    std::vector<kv> kvs;
    void* map = nullptr;
    size_t map_size = 0;
    bool open(const std::string& path);
    const gtensor* get(const std::string& name) const;
    int64_t key_i(const std::string& key, int64_t def) const;
    float key_f(const std::string& key, float def) const;
    const std::vector<int64_t>* key_arr(const std::string& key) const;
    ~gfile();
};

// ---- 4-bit tables in imi's 8-row layout (imi/core/tables.h:80-114, tables.cpp:67-97) ----
// per group of 8 rows and block of 32 columns: 128 B of codes (chunk t, bytes 4r..4r+3 = row r, columns 4t..4t+3
// low nibble, 16+4t..16+4t+3 high nibble), then fp16 scales [group][block][8]
struct q4tab {
    int rows = 0, cols = 0, nb = 0;
    bool has_m = false;            // Q4_1: weight = code * d + m (imi/core/tables.cpp:62,78-83)
    std::vector<uint8_t> codes;    // [rows/8][nb][128]
    std::vector<uint16_t> d;       // [rows/8][nb][8]
    std::vector<uint16_t> m;       // [rows/8][nb][8] (Q4_1 only)
};
// rows given as pointers to Q4_0 rows (nb blocks of 18 B: d, 16 B of nibbles) or, with q4_1, Q4_1 rows (20 B: d, m,
// 16 B of nibbles); rows.size() % 8 == 0
bool q4_build(q4tab& t, const std::vector<const uint8_t*>& rows, int cols, bool q4_1 = false);
int  q4_code_at(const uint8_t* blk128, int r, int k);   // imi/core/tables.cpp:167-169

// ---- activation cut to int8 per 32 (imi/core/vec.h:47-75) ----
float cut32(const float* x, int8_t* q, int* sum);          // d = amax/127, id = d ? 1/d : 0, q = rint(x*id)
struct q8in {                                              // imi_q8 (imi/core/tables.h:116-122, tables.cpp:100-109)
    int n = 0;
    std::vector<int8_t> q;
    std::vector<float> d, s;                               // per block: scale, scale * sum of codes
    void from(const float* x, int n);
};
struct q8b {                                               // imi_q8b, block-major (tables.cpp:405-416)
    int n = 0, cols = 0, nb = 0;
    std::vector<int8_t> q;                                 // [nb][n][32]
    std::vector<float> d, s;                               // [nb][n]
    void shape(int n_in, int n_cols);
    void set(int i, const float* x);
};

// ---- Q4 GEMV kernels (imi/core/tables.cpp:115-198, 419-477) ----
void q4_group(const q4tab& W, const q8in& X, int g, float* out);                                 // AVX2 op order
void q4_group2(const q4tab& W, const q8in& X, const q8in& X2, int g, float* out, float* out2);
void q4_group_batch(const q4tab& W, const q8b& X, int g, float* out);                            // out [n][8]
void q4_group_scalar(const q4tab& W, const q8in& X, int g, float* out);                          // same ops, scalar
void q4_block_sums(const q4tab& W, const q8in& X, int g, int32_t* sums);                         // [8][nb] integer sums

// ---- cfg-0 kernel: imi/kernels/q4x8.cpp ----
struct q4x8tab {                                            // imi/kernels/q4x8.h:8-12
    int rows = 0, cols = 0, nb = 0;
    std::vector<uint8_t> codes;    // [rows/8][nb][4][32]: byte i of chunk k = code(2k, i) | code(2k+1, i) << 4
    std::vector<float> scales;     // [rows/8][nb][8]
};
void q4x8_build(q4x8tab& t, const uint8_t* q4_0, int rows, int cols);            // q4x8.cpp:105-119
struct q4x8in { std::vector<int8_t> q; std::vector<float> d, corr; };            // q4x8.cpp:36
void q4x8_quant_in(const float* x, int n, q4x8in& o);                           // q4x8.cpp:38-48 (roundf)
void q4x8_rows(const q4x8tab& W, const q4x8in& X, float* y, int g0, int g1);     // q4x8.cpp:51-77

// ---- Q8_0 tables, k-major 8-row layout (imi/core/tables.cpp:289-402) ----
struct q8gtab {
    int rows = 0, rows_pad = 0, cols = 0, nb = 0;
    std::vector<int8_t> codes;     // [rows_pad/8][cols][8]
    std::vector<uint16_t> d;       // [rows_pad/8][nb][8]
};
bool q8g_build(q8gtab& t, const std::vector<const uint8_t*>& rows, int cols);
void q8g_group(const q8gtab& W, const float* xt, int C, int g, float* out);     // xt [cols][C] -> out [C][8]
void q8_0_dequant_row(const uint8_t* row, float* y, int cols);

// ---- Q6_K word table (imi/core/tables.cpp:200-287): 210-byte blocks of 256 values {ql[128], qh[64], scales[16], d} ----
struct q8kin {                                             // imi_q8k: the hidden state cut to int8 per 256 values
    int n = 0;
    std::vector<int8_t> q;
    std::vector<float> d;                                  // per 256: amax / 127
    std::vector<int16_t> bsums;                            // per 16 values: sum of their codes
    void from(const float* x, int n);                      // tables.cpp:200-213
};
int   q6k_at(const uint8_t* blk, int e);                   // value e (0..255) of a block, 0..63 (tables.cpp:215-233)
void  q6k_dequant_row(const uint8_t* row, float* y, int nblocks);                    // tables.cpp:216-233
void  q6k_lane_sums(const uint8_t* blk, const q8kin& X, int i, int32_t out[8]);      // block i's 8 int32 AVX2 lanes
float q6k_row(const uint8_t* row, const q8kin& X, int nblocks);                      // tables.cpp:235-277

// ---- small vector math (imi/core/vec.h:20-44) ----
float rms_scale(const float* x, int n, float eps);
void  norm_mul(const float* x, const float* w, float* o, int n, float eps);
void  norm_mul_add(const float* y, const float* w, float* x, int n, float eps);
void  rope(float* v, int n, int pos, float base, const float* ff);              // imi/core/seoul.cpp:19-28
float dot_h(const float* q, const uint16_t* k, int n);                          // seoul.cpp:29-39
void  axpy_h(float p, const uint16_t* v, float* o, int n);                      // seoul.cpp:40-47


}  // namespace orc
