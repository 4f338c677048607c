// Scratch memory of t0g_gemm_noalloc: a file-scope device array, so that
// entry point runs split-K without allocating (for callers that cannot call
// hipMalloc: code under HIP graph capture, serving loops, harnesses that
// forbid it).
//
// The array lives in this library's own code object (registered with the HIP
// runtime when libt0g.so loads); every GPU the library runs on holds its own
// copy, at its own address, until the process ends.  In host code the name
// `scratch` is only a host-side stand-in: its device address on a device is
// looked up with hipGetSymbolAddress, with that device current, once per
// device (t0g_device_open calls noalloc_scratch), and only that address is
// ever handed to kernels.
//
// Nothing in the array needs to start at zero: the split-K kernels write
// every element of the fp32 planes before the reduce kernel reads it.
#include <hip/hip_runtime.h>

#include <functional>
#include <mutex>

#include "t0g.h"
#include "t0g_internal.h"

// File scope, not in an anonymous namespace: the compiler then exports this
// static device variable from the device code object (under a name unique to
// this translation unit), which the HIP runtime needs to find it by name.
static __device__ __align__(256) unsigned char scratch[T0G_NOALLOC_SCRATCH_BYTES];

namespace {

constexpr int kMaxDevices = 64;
std::mutex g_mu;
uint64_t g_ptr[kMaxDevices];
// Per device: the event recorded after the last call that used the scratch, and
// the lock that makes "wait for it, launch, record it" one step, so calls from
// different handles or streams take the scratch one after another.
hipEvent_t g_last[kMaxDevices];
std::mutex g_use[kMaxDevices];

}  // namespace

namespace t0g {

int noalloc_scratch(int ordinal, uint64_t *ptr) {
    if (ordinal < 0 || ordinal >= kMaxDevices)
        return fail(T0G_ERR_INVALID_ARG, "device %d: the no-allocation scratch covers devices 0..%d", ordinal,
                    kMaxDevices - 1);
    std::lock_guard<std::mutex> lk(g_mu);
    if (!g_ptr[ordinal]) {
        void *p = nullptr;
        const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess || !p)
            return fail(T0G_ERR_HIP, "hipGetSymbolAddress(scratch) on device %d failed: %s (%d)", ordinal,
                        hipGetErrorString(e), (int)e);
        hipEvent_t ev = nullptr;
        const hipError_t e2 = hipEventCreateWithFlags(&ev, hipEventDisableTiming);
        if (e2 != hipSuccess)
            return fail(T0G_ERR_HIP, "hipEventCreateWithFlags (scratch order) on device %d failed: %s (%d)", ordinal,
                        hipGetErrorString(e2), (int)e2);
        g_last[ordinal] = ev;
        g_ptr[ordinal] = (uint64_t)p;
    }
    *ptr = g_ptr[ordinal];
    return T0G_OK;
}

int noalloc_scratch_use(int ordinal, hipStream_t stream, const std::function<int()> &launch) {
    std::lock_guard<std::mutex> lk(g_use[ordinal]);
    // Under stream capture the graph orders its own nodes; an event recorded outside
    // the capture cannot be waited for inside it, so the caller orders captured calls.
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    const bool capturing = hipStreamIsCapturing(stream, &cs) == hipSuccess && cs != hipStreamCaptureStatusNone;
    hipEvent_t ev = g_last[ordinal];
    if (!capturing) {
        const hipError_t e = hipStreamWaitEvent(stream, ev, 0);
        if (e != hipSuccess)
            return fail(T0G_ERR_HIP, "hipStreamWaitEvent (scratch order) failed: %s (%d)", hipGetErrorString(e), (int)e);
    }
    int rc = launch();
    if (rc || capturing) return rc;
    const hipError_t e = hipEventRecord(ev, stream);
    if (e != hipSuccess)
        return fail(T0G_ERR_HIP, "hipEventRecord (scratch order) failed: %s (%d)", hipGetErrorString(e), (int)e);
    return T0G_OK;
}

}  // namespace t0g
