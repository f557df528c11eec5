// Calibration launches for the measurements: the cost of an empty dispatch and of a pure read of a buffer the size of
// a table, each launched back to back on one stream, so a kernel's time can be set against what the dispatch path and
// HBM allow for the same bytes.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <string>
#include <vector>

#include "../../include/seoul_hip.h"

namespace sh {
int set_error(int code, const std::string& msg);
}
using namespace sh;

namespace {

__global__ __launch_bounds__(256) void k_empty(unsigned* out) {
    if (threadIdx.x > 1024) out[0] = 0;   // never true (256 threads): a dispatch with no work
}

// grid-stride read of n 16-byte words, 2 in flight per thread; one word of xor per workgroup (keeps the loads live).
// With st: thread 0 of each workgroup records the 100 MHz real-time clock at its start, when its first loads are back,
// and at its end.
__global__ __launch_bounds__(256) void k_read(const uint4* __restrict__ a, size_t n, unsigned* out, unsigned long long* st) {
    const unsigned long long t0 = __builtin_amdgcn_s_memrealtime();
    unsigned long long t1 = 0;
    const size_t stride = (size_t)gridDim.x * 512;
    unsigned acc = 0;
    for (size_t i = (size_t)blockIdx.x * 512 + threadIdx.x; i < n; i += stride) {
        const uint4 v0 = a[i];
        const uint4 v1 = i + 256 < n ? a[i + 256] : uint4{0, 0, 0, 0};
        acc ^= v0.x ^ v0.y ^ v0.z ^ v0.w ^ v1.x ^ v1.y ^ v1.z ^ v1.w;
        if (t1 == 0) t1 = __builtin_amdgcn_s_memrealtime() | 1;   // (after the loads' data is used)
    }
    for (int o = 32; o > 0; o >>= 1) acc ^= __shfl_xor(acc, o);
    __shared__ unsigned red[4];
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = acc;
    __syncthreads();
    if (threadIdx.x == 0) {
        out[blockIdx.x] = red[0] ^ red[1] ^ red[2] ^ red[3];
        if (st) {
            st[3 * blockIdx.x] = t0;
            st[3 * blockIdx.x + 1] = t1 ? t1 : t0;
            st[3 * blockIdx.x + 2] = __builtin_amdgcn_s_memrealtime();
        }
    }
}

// the XCD (accelerator complex die) each workgroup runs on: hardware register XCC_ID, read by the scalar unit
__global__ __launch_bounds__(64) void k_xcc(int* out) {
    unsigned v;
    asm volatile("s_getreg_b32 %0, hwreg(HW_REG_XCC_ID, 0, 4)" : "=s"(v));
    if (threadIdx.x == 0) out[blockIdx.x] = (int)v;
}

// one 72 KB slot per workgroup (512 threads x 9 x 16 B), slot (b + shift) % grid, ordinary (cached) or non-temporal
// loads; thread 0 records the workgroup's XCD
typedef unsigned u32x4c __attribute__((ext_vector_type(4)));
constexpr int L2_SLOT_WORDS = 4608;
__global__ __launch_bounds__(512) void k_pull(const u32x4c* base, int shift, int nt, unsigned* out, int* xid) {
    const int g = gridDim.x, b = (blockIdx.x + shift) % g;
    const u32x4c* p = base + (size_t)b * L2_SLOT_WORDS + threadIdx.x;
    u32x4c v[9];
    if (nt) {
#pragma unroll
        for (int q = 0; q < 9; q++) v[q] = __builtin_nontemporal_load(p + 512 * q);
    } else {
#pragma unroll
        for (int q = 0; q < 9; q++) v[q] = p[512 * q];
    }
    unsigned acc = 0;
#pragma unroll
    for (int q = 0; q < 9; q++) acc ^= v[q].x ^ v[q].y ^ v[q].z ^ v[q].w;
    if (acc == 0x9E3779B9u) out[blockIdx.x] = acc;   // (keeps the loads)
    if (threadIdx.x == 0) {
        unsigned x;
        asm volatile("s_getreg_b32 %0, hwreg(HW_REG_XCC_ID, 0, 4)" : "=s"(x));
        xid[blockIdx.x] = (int)x;
    }
}

#define KCHK(x)                                                                                                 \
    do {                                                                                                        \
        const hipError_t e_ = (x);                                                                              \
        if (e_ != hipSuccess) { err = e_; goto done; }                                                          \
    } while (0)

}  // namespace

extern "C" {

int sh_bench_empty(int device, int grid, int reps, double* us_per_launch) {
    if (grid < 1 || grid > 65536 || reps < 1 || !us_per_launch) return set_error(SH_E_ARG, "sh_bench_empty: bad argument");
    if (hipSetDevice(device) != hipSuccess) return set_error(SH_E_HIP, "sh_bench_empty: device");
    hipError_t err = hipSuccess;
    unsigned* out = nullptr;
    hipStream_t s = nullptr;
    hipEvent_t e0 = nullptr, e1 = nullptr;
    float ms = 0;
    KCHK(hipMalloc((void**)&out, 4));
    KCHK(hipStreamCreate(&s));
    KCHK(hipEventCreate(&e0));
    KCHK(hipEventCreate(&e1));
    for (int i = 0; i < 16; i++) hipLaunchKernelGGL(k_empty, dim3(grid), dim3(256), 0, s, out);
    KCHK(hipEventRecord(e0, s));
    for (int i = 0; i < reps; i++) hipLaunchKernelGGL(k_empty, dim3(grid), dim3(256), 0, s, out);
    KCHK(hipEventRecord(e1, s));
    KCHK(hipEventSynchronize(e1));
    KCHK(hipEventElapsedTime(&ms, e0, e1));
    *us_per_launch = 1e3 * ms / reps;
done:
    if (e0) (void)hipEventDestroy(e0);
    if (e1) (void)hipEventDestroy(e1);
    if (s) (void)hipStreamDestroy(s);
    if (out) (void)hipFree(out);
    return err == hipSuccess ? SH_OK : set_error(SH_E_HIP, std::string("sh_bench_empty: ") + hipGetErrorString(err));
}

int sh_bench_read(int device, long long bytes, int copies, int grid, int reps, double* us_per_launch, double* stamps) {
    if (bytes < 16 || bytes % 16 || copies < 1 || (long long)copies * bytes > (4ll << 30) || grid < 1 || grid > 65536 ||
        reps < 1 || !us_per_launch)
        return set_error(SH_E_ARG, "sh_bench_read: bad argument (bytes a multiple of 16, copies * bytes <= 4 GiB)");
    if (hipSetDevice(device) != hipSuccess) return set_error(SH_E_HIP, "sh_bench_read: device");
    hipError_t err = hipSuccess;
    uint4* a = nullptr;
    unsigned* out = nullptr;
    unsigned long long* st = nullptr;
    std::vector<unsigned long long> h;
    hipStream_t s = nullptr;
    hipEvent_t e0 = nullptr, e1 = nullptr;
    float ms = 0;
    const size_t n = (size_t)bytes / 16;
    KCHK(hipMalloc((void**)&a, (size_t)bytes * copies));
    KCHK(hipMemset(a, 1, (size_t)bytes * copies));
    KCHK(hipMalloc((void**)&out, (size_t)grid * 4));
    KCHK(hipStreamCreate(&s));
    KCHK(hipEventCreate(&e0));
    KCHK(hipEventCreate(&e1));
    KCHK(hipMalloc((void**)&st, (size_t)grid * 24));
    for (int c = 0; c < copies; c++)
        hipLaunchKernelGGL(k_read, dim3(grid), dim3(256), 0, s, a + (size_t)c * n, n, out, (unsigned long long*)nullptr);
    KCHK(hipEventRecord(e0, s));
    for (int r = 0; r < reps; r++)
        hipLaunchKernelGGL(k_read, dim3(grid), dim3(256), 0, s, a + (size_t)(r % copies) * n, n, out, (unsigned long long*)nullptr);
    KCHK(hipEventRecord(e1, s));
    KCHK(hipEventSynchronize(e1));
    KCHK(hipEventElapsedTime(&ms, e0, e1));
    *us_per_launch = 1e3 * ms / reps;
    if (stamps) {   // one more launch (the next copy in rotation, from HBM), stamped
        hipLaunchKernelGGL(k_read, dim3(grid), dim3(256), 0, s, a + (size_t)(reps % copies) * n, n, out, st);
        KCHK(hipStreamSynchronize(s));
        h.resize((size_t)3 * grid);
        KCHK(hipMemcpy(h.data(), st, h.size() * 8, hipMemcpyDeviceToHost));
        unsigned long long s0 = ~0ull, s0max = 0, emax = 0;
        std::vector<double> first;
        for (int g = 0; g < grid; g++) {
            s0 = std::min(s0, h[3 * g]);
            s0max = std::max(s0max, h[3 * g]);
            emax = std::max(emax, h[3 * g + 2]);
            first.push_back(0.01 * (double)(h[3 * g + 1] - h[3 * g]));
        }
        std::sort(first.begin(), first.end());
        stamps[0] = 0.01 * (double)(s0max - s0);        // last workgroup start, after the first
        stamps[1] = first[first.size() / 2];            // first loads back (median over workgroups)
        stamps[2] = 0.01 * (double)(emax - s0);         // last workgroup end, after the first start
    }
done:
    if (e0) (void)hipEventDestroy(e0);
    if (e1) (void)hipEventDestroy(e1);
    if (s) (void)hipStreamSynchronize(s), (void)hipStreamDestroy(s);
    if (out) (void)hipFree(out);
    if (st) (void)hipFree(st);
    if (a) (void)hipFree(a);
    return err == hipSuccess ? SH_OK : set_error(SH_E_HIP, std::string("sh_bench_read: ") + hipGetErrorString(err));
}

int sh_bench_xcc(int device, int grid, int launches, int* xcc) {
    if (grid < 1 || grid > 65536 || launches < 1 || launches > 64 || !xcc) return set_error(SH_E_ARG, "sh_bench_xcc: bad argument");
    if (hipSetDevice(device) != hipSuccess) return set_error(SH_E_HIP, "sh_bench_xcc: device");
    hipError_t err = hipSuccess;
    int* out = nullptr;
    hipStream_t s = nullptr;
    KCHK(hipMalloc((void**)&out, sizeof(int) * (size_t)grid * launches));
    KCHK(hipStreamCreate(&s));
    for (int l = 0; l < launches; l++) hipLaunchKernelGGL(k_xcc, dim3(grid), dim3(64), 0, s, out + (size_t)l * grid);
    KCHK(hipStreamSynchronize(s));
    KCHK(hipMemcpy(xcc, out, sizeof(int) * (size_t)grid * launches, hipMemcpyDeviceToHost));
done:
    if (s) (void)hipStreamSynchronize(s), (void)hipStreamDestroy(s);
    if (out) (void)hipFree(out);
    return err == hipSuccess ? SH_OK : set_error(SH_E_HIP, std::string("sh_bench_xcc: ") + hipGetErrorString(err));
}

int sh_bench_l2_reuse(int device, int pairs, double* us_second, double* us_alone, int* same_xcd) {
    if (pairs < 1 || pairs > 64 || !us_second || !us_alone || !same_xcd) return set_error(SH_E_ARG, "sh_bench_l2_reuse: bad argument");
    if (hipSetDevice(device) != hipSuccess) return set_error(SH_E_HIP, "sh_bench_l2_reuse: device");
    const int grid = 256;
    const size_t region = (size_t)grid * L2_SLOT_WORDS;   // 16-byte words: 18.9 MB
    hipError_t err = hipSuccess;
    u32x4c* buf = nullptr;
    unsigned* out = nullptr;
    int* xid = nullptr;
    hipStream_t s = nullptr;
    hipEvent_t e0 = nullptr, e1 = nullptr;
    std::vector<int> h(2 * grid);
    double t2 = 0, t1 = 0;
    int same = 0;
    KCHK(hipMalloc((void**)&buf, region * 16 * (size_t)(2 * pairs)));
    KCHK(hipMemset(buf, 1, region * 16 * (size_t)(2 * pairs)));
    KCHK(hipMalloc((void**)&out, 4 * grid));
    KCHK(hipMalloc((void**)&xid, sizeof(int) * 2 * grid));
    KCHK(hipStreamCreate(&s));
    KCHK(hipEventCreate(&e0));
    KCHK(hipEventCreate(&e1));
    for (int i = 0; i < pairs; i++) {
        float ms = 0;
        u32x4c* ra = buf + region * (size_t)(2 * i);
        u32x4c* rb = ra + region;
        // A then B over the same slots (workgroup b reads slot b in both), cached loads in both
        hipLaunchKernelGGL(k_pull, dim3(grid), dim3(512), 0, s, ra, 0, 0, out, xid);
        KCHK(hipEventRecord(e0, s));
        hipLaunchKernelGGL(k_pull, dim3(grid), dim3(512), 0, s, ra, 0, 0, out, xid + grid);
        KCHK(hipEventRecord(e1, s));
        KCHK(hipEventSynchronize(e1));
        KCHK(hipEventElapsedTime(&ms, e0, e1));
        t2 += ms;
        KCHK(hipMemcpy(h.data(), xid, sizeof(int) * 2 * grid, hipMemcpyDeviceToHost));
        for (int b = 0; b < grid; b++) same += h[b] == h[grid + b];
        // B alone on slots no launch has read
        KCHK(hipEventRecord(e0, s));
        hipLaunchKernelGGL(k_pull, dim3(grid), dim3(512), 0, s, rb, 0, 0, out, xid + grid);
        KCHK(hipEventRecord(e1, s));
        KCHK(hipEventSynchronize(e1));
        KCHK(hipEventElapsedTime(&ms, e0, e1));
        t1 += ms;
    }
    *us_second = 1e3 * t2 / pairs;
    *us_alone = 1e3 * t1 / pairs;
    *same_xcd = same;
done:
    if (e0) (void)hipEventDestroy(e0);
    if (e1) (void)hipEventDestroy(e1);
    if (s) (void)hipStreamSynchronize(s), (void)hipStreamDestroy(s);
    if (xid) (void)hipFree(xid);
    if (out) (void)hipFree(out);
    if (buf) (void)hipFree(buf);
    return err == hipSuccess ? SH_OK : set_error(SH_E_HIP, std::string("sh_bench_l2_reuse: ") + hipGetErrorString(err));
}

}  // extern "C"
