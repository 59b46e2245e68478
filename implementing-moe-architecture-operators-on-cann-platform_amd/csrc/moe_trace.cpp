// moe_trace.cpp -- per-kernel HIP-event timing (include/moe_trace.h).
//
// When enabled, each TraceScope records a start event before its kernel launch and a stop event after it,
// on the kernel's own stream. moe_trace_collect() waits for the pending stop events and folds the elapsed
// times into per-name totals. Events are recycled through a pool so a traced launch creates none once the
// pool is warm. When disabled a TraceScope costs one relaxed atomic load.
// The events are created with hipEventDisableSystemFence: they only time, and nothing reads memory through
// them, so recording one need not write back and invalidate the caches (which a default event does, at a cost
// of a few µs of GPU time per record and colder caches for the kernel that follows).

#include <hip/hip_runtime.h>

#include <atomic>
#include <mutex>
#include <string>
#include <vector>

#include "moe_launch.h"
#include "moe_trace.h"

namespace {

struct Pending {
    const char* name;
    hipEvent_t start;
    hipEvent_t stop;
};

struct Total {
    std::string name;
    int64_t launches;
    double ms;
};

std::atomic<bool> g_on{false};
std::mutex g_mu;
std::vector<Pending> g_pending;
std::vector<Total> g_totals;
std::vector<hipEvent_t> g_pool;

hipEvent_t take_event() {
    {
        std::lock_guard<std::mutex> lock(g_mu);
        if (!g_pool.empty()) {
            hipEvent_t ev = g_pool.back();
            g_pool.pop_back();
            return ev;
        }
    }
    hipEvent_t ev = nullptr;
    if (hipEventCreateWithFlags(&ev, hipEventDisableSystemFence) != hipSuccess) return nullptr;
    return ev;
}

void give_event_locked(hipEvent_t ev) {
    if (ev) g_pool.push_back(ev);
}

void drop_pending_locked() {
    for (auto& p : g_pending) {
        (void)hipEventSynchronize(p.stop);
        give_event_locked(p.start);
        give_event_locked(p.stop);
    }
    g_pending.clear();
}

}  // namespace

namespace moe {

TraceScope::TraceScope(const char* name, hipStream_t stream) : name_(name), stream_(stream) {
    if (!g_on.load(std::memory_order_relaxed)) return;
    start_ = take_event();
    if (start_ && hipEventRecord(start_, stream_) != hipSuccess) {
        std::lock_guard<std::mutex> lock(g_mu);
        give_event_locked(start_);
        start_ = nullptr;
    }
}

TraceScope::~TraceScope() {
    if (!start_) return;
    hipEvent_t stop = take_event();
    std::lock_guard<std::mutex> lock(g_mu);
    if (!stop || hipEventRecord(stop, stream_) != hipSuccess) {
        give_event_locked(stop);
        give_event_locked(start_);
        return;
    }
    g_pending.push_back(Pending{name_, start_, stop});
}

}  // namespace moe

extern "C" {

moe_status moe_trace_enable(int32_t on) {
    std::lock_guard<std::mutex> lock(g_mu);
    if (on) {
        drop_pending_locked();
        g_totals.clear();
    }
    g_on.store(on != 0, std::memory_order_relaxed);
    return MOE_OK;
}

int32_t moe_trace_collect(void) {
    std::lock_guard<std::mutex> lock(g_mu);
    for (auto& p : g_pending) {
        float ms = 0.0f;
        if (hipEventSynchronize(p.stop) == hipSuccess && hipEventElapsedTime(&ms, p.start, p.stop) == hipSuccess) {
            Total* t = nullptr;
            for (auto& q : g_totals)
                if (q.name == p.name) t = &q;
            if (!t) {
                g_totals.push_back(Total{p.name, 0, 0.0});
                t = &g_totals.back();
            }
            t->launches += 1;
            t->ms += ms;
        }
    }
    drop_pending_locked();  // every stop event has completed: recycle them
    return static_cast<int32_t>(g_totals.size());
}

moe_status moe_trace_get(int32_t index, const char** name, int64_t* launches, double* total_ms) {
    std::lock_guard<std::mutex> lock(g_mu);
    if (index < 0 || index >= static_cast<int32_t>(g_totals.size())) return MOE_ERR_ARG;
    if (name) *name = g_totals[static_cast<size_t>(index)].name.c_str();
    if (launches) *launches = g_totals[static_cast<size_t>(index)].launches;
    if (total_ms) *total_ms = g_totals[static_cast<size_t>(index)].ms;
    return MOE_OK;
}

}  // extern "C"
