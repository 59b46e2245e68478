// moe_noalloc.hip -- the fixed device scratch behind moe_expert_ffn_no_alloc (include/moe_ops.h).
//
// Callers that cannot allocate device memory (code under HIP graph capture, tight serving loops, harnesses that
// forbid hipMalloc) get the FFN's workspace from one file-scope device array instead of a caller buffer. Each
// GPU the library runs on holds its own copy of the array (kScratchBytes) until the process ends. Host code never
// passes the array's name to a kernel (on the host it is only a stand-in symbol); it looks up the array's device
// address once per device, with that device current, and passes that address.
//
// Every call on a GPU shares that GPU's array and it keeps the last call's contents; the FFN writes every
// workspace byte it later reads (offsets, sorted slots, the SwiGLU intermediate, split partials), so nothing
// needs clearing between calls. Calls that overlap on one GPU (two streams, two threads) race on the array.

#include <hip/hip_runtime.h>

#include <mutex>
#include <vector>

#include "moe_launch.h"

namespace moe {

namespace {

constexpr size_t kScratchBytes = size_t(64) << 20;  // 64 MiB per GPU

static __device__ __align__(256) uint8_t scratch[kScratchBytes];

struct DeviceScratch {
    int device;
    void* ptr;
};

std::mutex g_mu;
std::vector<DeviceScratch> g_scratch;

}  // namespace

size_t noalloc_scratch_bytes() { return kScratchBytes; }

hipError_t noalloc_scratch(void** ptr) {
    int dev = 0;
    hipError_t err = hipGetDevice(&dev);
    if (err != hipSuccess) return err;
    std::lock_guard<std::mutex> lock(g_mu);
    for (const DeviceScratch& d : g_scratch) {
        if (d.device == dev) {
            *ptr = d.ptr;
            return hipSuccess;
        }
    }
    void* addr = nullptr;
    err = hipGetSymbolAddress(&addr, HIP_SYMBOL(scratch));
    if (err != hipSuccess || addr == nullptr) {
        (void)hipGetLastError();  // leave no sticky error for later calls
        return err != hipSuccess ? err : hipErrorInvalidSymbol;
    }
    g_scratch.push_back(DeviceScratch{dev, addr});
    *ptr = addr;
    return hipSuccess;
}

}  // namespace moe
