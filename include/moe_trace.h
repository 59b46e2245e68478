/*
 * moe_trace.h -- per-kernel GPU timing inside libmoe_mi355x.so.
 *
 * No counterpart in the reference, which times whole operator chains with host std::chrono only
 * (tests/test_moe.cpp:590-612, tests/moe_cpu_sim.cpp:629-640). When enabled, the library records a HIP event
 * pair around every kernel it launches, on the stream that kernel is launched on, and accumulates the
 * elapsed times per kernel name. Disabled by default; enabling it adds two event records per launch. The
 * events carry no system-scope fence (timing only), so recording them flushes no cache.
 * The tracer is process-global and guarded by a mutex.
 */
#ifndef MOE_TRACE_H
#define MOE_TRACE_H

#include <stdint.h>
#include "moe_ops.h"

#ifdef __cplusplus
extern "C" {
#endif

/* Turn event recording on (1) or off (0). Turning it on clears earlier results. */
moe_status moe_trace_enable(int32_t on);
/* Wait for all recorded events, fold them into the per-kernel totals and return the number of kernels seen. */
int32_t moe_trace_collect(void);
/* Totals of kernel `index` (0 <= index < moe_trace_collect()). *name stays valid until the next enable. */
moe_status moe_trace_get(int32_t index, const char** name, int64_t* launches, double* total_ms);

#ifdef __cplusplus
}
#endif

#endif /* MOE_TRACE_H */
