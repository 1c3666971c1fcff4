// exl3c4_noalloc.hip -- exl3c4_launch_noalloc: exl3c4_launch with the library's own scratch, for callers that cannot
// allocate (code under HIP graph capture, tight serving loops, harnesses that forbid hipMalloc). No counterpart in the
// reference.
//
// The scratch is one file-scope device array, `scratch`, of EXL3C4_NOALLOC_SCRATCH_BYTES: each GPU the library runs on
// holds its own copy at its own address until the process ends. In host code the array's name is only a host-side
// stand-in (passing it to a kernel compiles and then faults), so the first call on a device, with that device
// current, asks the runtime for the device address once (hipGetSymbolAddress) and keeps it per device; every use
// after that -- the launch's kernel arguments -- takes that address. Nothing here allocates: the launch it hands over
// to (exl3c4_launch) allocates nothing either, and zeroes what must start at zero (gate_up_down's counters) with a
// fill kernel of its own.
//
// Every call on one GPU shares that GPU's array and leaves the last call's contents in it: two calls that may overlap
// on one GPU (two streams, or two threads) race and must be ordered by the caller.
#include <hip/hip_runtime.h>

#include <mutex>

#include "exl3c4_dev.h"

namespace {

static __device__ __align__(256) unsigned char scratch[EXL3C4_NOALLOC_SCRATCH_BYTES];

constexpr int kMaxDevices = 64;
std::once_flag g_once[kMaxDevices];
void*          g_ptr[kMaxDevices];
hipError_t     g_err[kMaxDevices];

// The device address of this device's array: asked for once per device, with the device current.
void* scratch_of(int dev) {
    std::call_once(g_once[dev], [dev] {
        void* p = nullptr;
        g_err[dev] = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        g_ptr[dev] = g_err[dev] == hipSuccess ? p : nullptr;
    });
    return g_ptr[dev];
}

}  // namespace

extern "C" int64_t exl3c4_noalloc_scratch_bytes(void) { return EXL3C4_NOALLOC_SCRATCH_BYTES; }

extern "C" int exl3c4_launch_noalloc(const Exl3c4Op* op, void* stream) {
    if (!op) return EXL3C4_E_INVAL;
    const int64_t need = exl3c4_launch_scratch_bytes(op);        // the op's own refusals first
    if (need < 0) return (int)need;
    if (need > EXL3C4_NOALLOC_SCRATCH_BYTES) return EXL3C4_E_SCRATCH;
    int dev = -1;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return EXL3C4_E_DEVICE;
    if (stream) {                                                 // the array used is the current device's
        hipDevice_t sdev = -1;
        if (hipStreamGetDevice((hipStream_t)stream, &sdev) != hipSuccess || sdev != dev) return EXL3C4_E_DEVICE;
    }
    void* s = scratch_of(dev);
    if (!s) return EXL3C4_E_DEVICE;
    return exl3c4_launch(op, s, EXL3C4_NOALLOC_SCRATCH_BYTES, stream);
}
