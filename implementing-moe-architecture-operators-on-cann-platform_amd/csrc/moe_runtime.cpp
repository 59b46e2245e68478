// moe_runtime.cpp -- per-device launch preparation shared by the kernel files (moe_launch.h).
//
// Kernel attributes and occupancy are properties of a kernel on one device: a process that launches on several
// GPUs must set the dynamic-LDS limit on each of them. Both are cached in small mutex-guarded tables keyed by
// (device, kernel[, LDS bytes]); a launch after the first costs one lookup.

#include <hip/hip_runtime.h>

#include <mutex>
#include <vector>

#include "moe_launch.h"

namespace moe {

namespace {

struct LdsLimit {
    int device;
    const void* fn;
    int bytes;
};

struct Resident {
    int device;
    const void* fn;
    int threads;
    size_t lds;
    int workgroups;
};

std::mutex g_mu;
std::vector<LdsLimit> g_limits;
std::vector<Resident> g_resident;

}  // namespace

hipError_t ensure_lds_limit(const void* fn, int lds_max) {
    int dev = 0;
    hipError_t err = hipGetDevice(&dev);
    if (err != hipSuccess) return err;
    std::lock_guard<std::mutex> lock(g_mu);
    for (const LdsLimit& l : g_limits)
        if (l.device == dev && l.fn == fn && l.bytes >= lds_max) return hipSuccess;
    err = hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, lds_max);
    if (err != hipSuccess) {
        (void)hipGetLastError();  // leave no sticky error for later calls
        return err;
    }
    g_limits.push_back(LdsLimit{dev, fn, lds_max});
    return hipSuccess;
}

int resident_workgroups(const void* fn, int threads, size_t lds) {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) return 0;
    std::lock_guard<std::mutex> lock(g_mu);
    for (const Resident& r : g_resident)
        if (r.device == dev && r.fn == fn && r.threads == threads && r.lds == lds) return r.workgroups;
    int cus = 0, per_cu = 0;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
        hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, fn, threads, lds) != hipSuccess) {
        (void)hipGetLastError();
        return 0;
    }
    const int n = cus * (per_cu > 0 ? per_cu : 1);
    g_resident.push_back(Resident{dev, fn, threads, lds, n});
    return n;
}

}  // namespace moe
