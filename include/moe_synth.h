/*
 * moe_synth.h -- synthetic-input and calibration helpers of libmoe_mi355x.so, used by bench.py and the tests.
 *
 * No counterpart on the reference's operator path: the reference generates its inputs on the host
 * (tests/moe_cpu_sim.cpp:161-167, tests/test_moe.cpp:373-381). These fill large device tensors in place so
 * that gigabyte-sized expert weights need not cross PCIe.
 */
#ifndef MOE_SYNTH_H
#define MOE_SYNTH_H

#include <stdint.h>
#include "moe_ops.h"

#ifdef __cplusplus
extern "C" {
#endif

/*
 * Fill out[0, n) with fp16 samples of N(0, sigma_i^2), sigma_i = (i % period) < split ? sigma_a : sigma_b.
 * Element i is a pure function of (seed, stream_id, i):
 *   key = mix64(seed * 0x9E3779B97F4A7C15 + stream_id * 0xD1B54A32D192ED03 + 0x632BE59BD9B4E019)
 *   z   = mix64(key + (i + 1) * 0x9E3779B97F4A7C15)            (all arithmetic mod 2^64)
 *   mix64(z): z = (z ^ z>>30) * 0xBF58476D1CE4E5B9; z = (z ^ z>>27) * 0x94D049BB133111EB; z ^ z>>31
 *   u1 = ((z >> 32) + 0.5) * 2^-32, u2 = ((z & 0xFFFFFFFF) + 0.5) * 2^-32
 *   n  = sqrt(-2 ln u1) * cos(2 pi u2)                           (Box-Muller, binary64)
 *   out[i] = fp16_round_nearest_even(n * sigma_i)                (one rounding from binary64)
 * The numpy mirror in the package's synth.py implements the same function.
 */
moe_status moe_synth_normal_f16(uint16_t* out, uint64_t n, uint64_t seed, uint64_t stream_id, double sigma_a,
                                double sigma_b, uint64_t period, uint64_t split, void* stream);

/* Plain device copy of `bytes` bytes (multiple of 16, 16-byte aligned) used to calibrate HBM counters. */
moe_status moe_copy_bytes(void* dst, const void* src, uint64_t bytes, void* stream);

/* Read `bytes` bytes (multiple of 16384, 16-byte aligned) with whole-line non-temporal loads and discard them:
 * the achievable HBM read rate of this device, reported beside the published peak. */
moe_status moe_stream_read_bytes(const void* src, uint64_t bytes, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* MOE_SYNTH_H */
