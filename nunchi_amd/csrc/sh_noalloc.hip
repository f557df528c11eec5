// The kernel-level batch product (sh_q4_gemm) for callers that cannot allocate device memory: code under HIP
// graph capture, serving loops with a fixed memory budget. Its one work buffer, the int8 cut of the input
// (block-major codes, scales and d * sum per 32 columns), lives in a fixed array of device memory, one copy per
// device, held until the process ends. Every call on a device uses that device's copy: calls of one context are
// ordered by its stream, and a call from another context than the device's last user first waits (on its own stream)
// for an event recorded after that last call, so contexts on one device do not overwrite each other's cut. Each call's
// cut kernel writes every entry its product reads, so nothing needs clearing between calls. Under graph capture of
// the context's stream no event is recorded or waited for: calls from two contexts captured into graphs that replay
// at the same time on one device race.
#include <hip/hip_runtime.h>

#include <mutex>
#include <string>

#include "sh_ctx.h"
#include "sh_prefill.h"

namespace sh {
namespace {

constexpr size_t NA_MAX_CODES = size_t(1) << 20;                    // n * cols int8 codes at most
constexpr size_t NA_SCALE_BYTES = (NA_MAX_CODES / 32) * sizeof(float);
constexpr size_t NA_BYTES = NA_MAX_CODES + 2 * NA_SCALE_BYTES;       // codes, then d, then s

static __device__ __align__(256) unsigned char scratch[NA_BYTES];

constexpr int NA_MAX_DEVICES = 64;
std::mutex g_mu;
unsigned char* g_ptr[NA_MAX_DEVICES] = {};   // the array's address on each device (0 until set up)
hipEvent_t g_ev[NA_MAX_DEVICES] = {};        // recorded after each call on the device
const sh_ctx* g_last[NA_MAX_DEVICES] = {};   // the context of that call (compared only, never dereferenced)

}  // namespace

// Find the array's address on `device`, which must be the current device. Called once per context creation; the
// address is looked up once per device and kept.
int noalloc_setup(int device) {
    if (device < 0 || device >= NA_MAX_DEVICES) return set_error(SH_E_ARG, "noalloc: device index above 63");
    std::lock_guard<std::mutex> lk(g_mu);
    if (g_ptr[device]) return SH_OK;
    void* p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p) return set_error(SH_E_HIP, std::string("noalloc: hipGetSymbolAddress: ") + hipGetErrorString(e));
    hipEvent_t ev = nullptr;
    const hipError_t ee = hipEventCreateWithFlags(&ev, hipEventDisableTiming);
    if (ee != hipSuccess) return set_error(SH_E_HIP, std::string("noalloc: hipEventCreate: ") + hipGetErrorString(ee));
    g_ptr[device] = static_cast<unsigned char*>(p);
    g_ev[device] = ev;
    return SH_OK;
}

}  // namespace sh

using namespace sh;

extern "C" int sh_q4_gemm_noalloc(sh_ctx* c, const sh_q4* t, const float* x_dev, int n, float* y_dev) {
    if (!c || !t || !x_dev || !y_dev || n < 1 || n > PF_MAX_N) return set_error(SH_E_ARG, "sh_q4_gemm_noalloc: bad argument (1 <= n <= 512)");
    if (t->ctx != c) return set_error(SH_E_STATE, "sh_q4_gemm_noalloc: table belongs to another context");
    const q4dev& W = t->t;
    const size_t codes = (size_t)n * W.cols;
    if (codes > NA_MAX_CODES)
        return set_error(SH_E_ARG, "sh_q4_gemm_noalloc: n * cols = " + std::to_string(codes) + " is above the scratch maximum of " +
                                       std::to_string(NA_MAX_CODES));
    // (the lock is held over the wait, both launches and the record, so two threads' calls cannot interleave)
    std::lock_guard<std::mutex> lk(g_mu);
    const int dev = c->device;
    unsigned char* base = (dev >= 0 && dev < NA_MAX_DEVICES) ? g_ptr[dev] : nullptr;
    if (!base) return set_error(SH_E_STATE, "sh_q4_gemm_noalloc: no scratch on this context's device");
    hipError_t e = hipSetDevice(dev);
    hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
    if (e == hipSuccess) e = hipStreamIsCapturing(c->stream, &cap);
    const bool capturing = cap != hipStreamCaptureStatusNone;
    // another context's call may still be reading the scratch: this stream waits for it
    if (e == hipSuccess && !capturing && g_last[dev] && g_last[dev] != c) e = hipStreamWaitEvent(c->stream, g_ev[dev], 0);
    const pf_cut cut{reinterpret_cast<int8_t*>(base), reinterpret_cast<float*>(base + NA_MAX_CODES),
                     reinterpret_cast<float*>(base + NA_MAX_CODES + NA_SCALE_BYTES)};
    if (e == hipSuccess) e = launch_pf_cut(pf_cutk_args{x_dev, W.cols, W.cols, n, cut}, c->stream);
    pf_gemm_args g{};
    g.W = W;
    g.n = n;
    g.in = cut;
    g.out = y_dev;
    g.out_ld = W.rows;
    if (e == hipSuccess) e = launch_pf_gemm(EPI_STORE, g, c->stream);
    if (e == hipSuccess && !capturing) {
        e = hipEventRecord(g_ev[dev], c->stream);
        if (e == hipSuccess) g_last[dev] = c;
    }
    if (e != hipSuccess) return set_error(SH_E_HIP, std::string("sh_q4_gemm_noalloc: ") + hipGetErrorString(e));
    return SH_OK;
}
