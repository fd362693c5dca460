// Fixed device scratch for ifr_matmul_quant_noalloc: the quantized copy of
// the GEMV's input vector lives in a file-scope device array instead of a
// buffer the library allocates, so the entry point never calls hipMalloc.
//
// Each GPU holds its own instance of the array (for as long as the process
// lives).  Host code never passes the array's name to a kernel: in host code
// it is a stand-in, not a device address.  ifr_noalloc_init looks up the
// device address once per device with hipGetSymbolAddress, with that device
// current, and every use goes through the pointer it returns.
#include <hip/hip_runtime.h>

#include <mutex>

#include "noalloc.h"

static __device__ __align__(256) uint8_t scratch[IFR_NOALLOC_SCRATCH_BYTES];

namespace {
constexpr int MAX_DEVICES = 64;
std::mutex g_mu;
void *g_ptr[MAX_DEVICES] = {};
} // namespace

// The caller has made `device` current.  Returns hipSuccess and the device
// address of this device's array.
hipError_t ifr_noalloc_init(int device, void **ptr) {
    if (device < 0 || device >= MAX_DEVICES || !ptr) return hipErrorInvalidValue;
    std::lock_guard<std::mutex> lock(g_mu);
    if (!g_ptr[device]) {
        void *p = nullptr;
        const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess) return e;
        g_ptr[device] = p;
    }
    *ptr = g_ptr[device];
    return hipSuccess;
}
