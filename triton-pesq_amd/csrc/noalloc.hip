// Forward pass of the loss that allocates nothing (pesq_pipeline_forward_noalloc).
//
// Callers that cannot allocate device memory (code under HIP graph capture,
// tight serving loops, harnesses that forbid hipMalloc) pass only inputs and
// outputs.  The forward workspace is a static device array of this file,
// `scratch`, which each GPU the library runs on holds until the process ends.
// Its device address comes from hipGetSymbolAddress, once per device with that
// device current, on the entry point's first call there; the host-side name of
// the array is never used as a device address.
//
// Every call on one GPU shares that GPU's array: calls that overlap on one GPU
// (on different streams, or from different threads without ordering) race and
// must not be issued.  The forward pass writes every workspace value before it
// reads it (no region needs clearing between calls), so back-to-back calls on
// one stream are safe and give the same results as pesq_pipeline_forward.
#include <atomic>
#include <mutex>

#include "common.hpp"

namespace pesq {

constexpr size_t kScratchBytes = PESQ_NOALLOC_SCRATCH_BYTES;
constexpr int kMaxDevices = 64;

static __device__ __align__(256) unsigned char scratch[kScratchBytes];

static std::atomic<void *> g_scratch_ptr[kMaxDevices];
static std::mutex g_scratch_mutex;

// Device address of `scratch` on `device`, looked up on first use.
static int scratch_address(int device, void **out) {
    PESQ_CHECK_ARG(device >= 0 && device < kMaxDevices, "device %d out of range", device);
    void *ptr = g_scratch_ptr[device].load(std::memory_order_acquire);
    if (ptr != nullptr) {
        *out = ptr;
        return PESQ_OK;
    }
    std::lock_guard<std::mutex> lock(g_scratch_mutex);
    ptr = g_scratch_ptr[device].load(std::memory_order_relaxed);
    if (ptr == nullptr) {
        int current = -1;
        hipError_t err = hipGetDevice(&current);
        if (err == hipSuccess && current != device) err = hipSetDevice(device);
        if (err == hipSuccess) err = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
        if (current >= 0 && current != device) {
            const hipError_t restore = hipSetDevice(current);
            if (err == hipSuccess) err = restore;
        }
        if (err != hipSuccess || ptr == nullptr) {
            set_error("hipGetSymbolAddress(scratch) on device %d: %s", device,
                      hipGetErrorString(err));
            return PESQ_ERR_HIP;
        }
        g_scratch_ptr[device].store(ptr, std::memory_order_release);
    }
    *out = ptr;
    return PESQ_OK;
}

}  // namespace pesq

using namespace pesq;

extern "C" int pesq_pipeline_forward_noalloc(const float *ref, const float *deg, int64_t batch,
                                             int64_t len, const void *model_table, double factor,
                                             float *d_symm, float *d_asymm, float *mos,
                                             float *loss, hipStream_t stream) {
    size_t bytes = 0;
    if (int st = pesq_pipeline_forward_workspace(batch, len, 0, &bytes)) return st;
    PESQ_CHECK_ARG(bytes <= kScratchBytes,
                   "pesq_pipeline_forward_noalloc: %lld x %lld samples need %zu bytes of "
                   "workspace, more than the %zu bytes of its static scratch; use "
                   "pesq_pipeline_forward with a workspace",
                   (long long)batch, (long long)len, bytes, kScratchBytes);
    int device = -1;
    hipError_t err = hipStreamGetDevice(stream, &device);
    if (err != hipSuccess) {
        set_error("hipStreamGetDevice: %s", hipGetErrorString(err));
        return PESQ_ERR_HIP;
    }
    void *ws = nullptr;
    if (int st = scratch_address(device, &ws)) return st;
    return pesq_pipeline_forward(ref, deg, batch, len, model_table, factor, 0, d_symm, d_asymm,
                                 mos, loss, ws, stream);
}
