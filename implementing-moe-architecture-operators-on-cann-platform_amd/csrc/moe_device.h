// moe_device.h -- types and helpers shared by the gfx950 kernels of libmoe_mi355x.so.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace moe {

typedef _Float16 f16;
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

constexpr int kWave = 64;  // CDNA wavefront width

// 16-byte global load of 8 fp16 values (address must be 16-byte aligned).
__device__ __forceinline__ f16x8 load_f16x8(const uint16_t* p) {
    return *reinterpret_cast<const f16x8*>(p);
}

// Same, marked non-temporal: used for expert weights that are streamed exactly once per layer, so they do
// not evict the token rows that every workgroup of an expert re-reads from L2.
__device__ __forceinline__ f16x8 load_f16x8_stream(const uint16_t* p) {
    u32x4 v = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p));
    return __builtin_bit_cast(f16x8, v);
}

__device__ __forceinline__ uint16_t f32_to_f16_bits(float v) {
    return __builtin_bit_cast(uint16_t, static_cast<f16>(v));  // v_cvt_f16_f32, round to nearest even
}

__device__ __forceinline__ float f16_bits_to_f32(uint16_t b) {
    return static_cast<float>(__builtin_bit_cast(f16, b));
}

// D(16x16, fp32) += A(16x32, fp16) * B(32x16, fp16).
// Lane l supplies A row (l % 16) and B column (l % 16), each as 8 consecutive k of the k-group (l / 16); any
// bijection of the 32 k values works as long as A and B use the same one. D comes back as
// D[4 * (l / 16) + r][l % 16] in element r of lane l.
__device__ __forceinline__ f32x4 mfma16x16x32(f16x8 a, f16x8 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ int lane_id() { return static_cast<int>(threadIdx.x) & (kWave - 1); }

// s_waitcnt immediate that waits until at most n (< 64) vector-memory operations of this wave are outstanding
// (gfx9 encoding: vmcnt bits [3:0] and [15:14]; lgkmcnt and expcnt left at their maximum, i.e. not waited on).
constexpr unsigned vmcnt_imm(int n) { return 0x0f70u | (n & 15) | ((n >> 4) << 14); }

// SwiGLU of one fp32 (gate, up) pair: silu(g) * u = g / (1 + exp(-g)) * u. Contraction into FMAs is off, so each
// operation rounds on its own and the result does not depend on how the compiler schedules the code around it
// (with contraction on, unrolled copies of the same epilogue were seen to round differently).
__device__ __forceinline__ float swiglu_f32(float g, float u) {
#pragma clang fp contract(off)
    const float silu = g / (1.0f + expf(-g));
    return silu * u;
}

}  // namespace moe
