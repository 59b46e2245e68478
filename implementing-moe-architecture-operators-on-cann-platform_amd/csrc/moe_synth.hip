// moe_synth.hip -- synthetic fp16 normal samples and a plain copy kernel (bench / test utilities).
//
// The generator is a counter-based hash (splitmix64 finaliser) feeding Box-Muller in binary64, then one
// rounding to fp16; the numpy mirror in synth.py computes the same function. Contraction is disabled so
// each binary64 operation rounds exactly as numpy's does.

#include "moe_device.h"
#include "moe_launch.h"

#pragma clang fp contract(off)

namespace moe {

__device__ u32x4 g_read_sink;  // written only by stream_read_kernel, on a value its data never takes

namespace {

constexpr uint64_t kGolden = 0x9E3779B97F4A7C15ull;

__host__ __device__ __forceinline__ uint64_t mix64(uint64_t z) {
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

// binary64 -> binary16, round to nearest even, in one step (no intermediate binary32 rounding).
__device__ __forceinline__ uint16_t f64_to_f16_rne(double d) {
    const uint64_t b = __builtin_bit_cast(uint64_t, d);
    const uint16_t sign = static_cast<uint16_t>((b >> 48) & 0x8000u);
    const int exp = static_cast<int>((b >> 52) & 0x7FF);
    const uint64_t mant = b & ((uint64_t{1} << 52) - 1);
    if (exp == 0x7FF) return static_cast<uint16_t>(sign | 0x7C00u | (mant ? 0x200u : 0u));
    const int e = exp - 1023;
    if (e > 15) return static_cast<uint16_t>(sign | 0x7C00u);
    uint64_t sig;
    int shift;
    uint32_t hexp;
    if (e >= -14) {  // normal binary16 range
        sig = mant;
        shift = 42;
        hexp = static_cast<uint32_t>(e + 15) << 10;
    } else {  // subnormal binary16 (or zero): value = sig * 2^-24 after the shift
        if (exp == 0) return sign;  // binary64 zero / subnormal -> signed zero
        sig = mant | (uint64_t{1} << 52);
        shift = 42 + (-14 - e);
        if (shift > 63) return sign;
        hexp = 0;
    }
    uint64_t q = sig >> shift;
    const uint64_t rem = sig & ((uint64_t{1} << shift) - 1);
    const uint64_t half = uint64_t{1} << (shift - 1);
    if (rem > half || (rem == half && (q & 1))) q += 1;
    return static_cast<uint16_t>(sign | static_cast<uint16_t>(hexp + q));  // a mantissa carry rolls into exp
}

__global__ void synth_normal_kernel(uint16_t* __restrict__ out, uint64_t n, uint64_t key, double sa, double sb,
                                    uint64_t period, uint64_t split) {
    const uint64_t stride = static_cast<uint64_t>(gridDim.x) * blockDim.x;
    for (uint64_t i = static_cast<uint64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < n; i += stride) {
        const uint64_t z = mix64(key + (i + 1) * kGolden);
        const double u1 = (static_cast<double>(z >> 32) + 0.5) * 0x1p-32;
        const double u2 = (static_cast<double>(z & 0xFFFFFFFFull) + 0.5) * 0x1p-32;
        const double r = sqrt(-2.0 * log(u1));
        const double nv = r * cos(6.283185307179586 * u2);
        const double sigma = (i % period) < split ? sa : sb;
        out[i] = f64_to_f16_rne(nv * sigma);
    }
}

__global__ void copy_kernel(u32x4* __restrict__ dst, const u32x4* __restrict__ src, uint64_t n16) {
    const uint64_t stride = static_cast<uint64_t>(gridDim.x) * blockDim.x;
    for (uint64_t i = static_cast<uint64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < n16; i += stride)
        dst[i] = src[i];
}

// Achievable HBM read rate: each wave reads contiguous 16 KB pieces as 16 non-temporal loads of 1 KB (64 lanes x
// 16 B), all in flight before use; pieces are dealt grid-stride. The xor of the data goes to a sink only if it
// equals a value it never takes, which keeps the loads (the sink has external linkage, so the store is
// observable and cannot be dropped).
__global__ __launch_bounds__(512) void stream_read_kernel(const u32x4* __restrict__ src, uint64_t pieces) {
    const uint64_t waves = static_cast<uint64_t>(gridDim.x) * (blockDim.x / 64);
    const int lane = static_cast<int>(threadIdx.x) & 63;
    u32x4 acc = {0u, 0u, 0u, 0u};
    for (uint64_t pc = static_cast<uint64_t>(blockIdx.x) * (blockDim.x / 64) + threadIdx.x / 64; pc < pieces;
         pc += waves) {
        const u32x4* base = src + pc * 1024 + lane;
        u32x4 v[16];
#pragma unroll
        for (int j = 0; j < 16; ++j) v[j] = __builtin_nontemporal_load(base + j * 64);
#pragma unroll
        for (int j = 0; j < 16; ++j) acc ^= v[j];
    }
    if ((acc.x & acc.y & acc.z & acc.w) == 0xfeedf00du) g_read_sink = acc;
}

}  // namespace

hipError_t launch_synth_normal_f16(uint16_t* out, uint64_t n, uint64_t seed, uint64_t stream_id, double sigma_a,
                                   double sigma_b, uint64_t period, uint64_t split, hipStream_t stream) {
    const uint64_t key = mix64(seed * kGolden + stream_id * 0xD1B54A32D192ED03ull + 0x632BE59BD9B4E019ull);
    const uint64_t blocks = (n + 255) / 256;
    const int grid = static_cast<int>(blocks < 16384 ? (blocks ? blocks : 1) : 16384);
    TraceScope trace("moe_synth_normal_f16", stream);
    synth_normal_kernel<<<grid, 256, 0, stream>>>(out, n, key, sigma_a, sigma_b, period ? period : 1, split);
    return hipGetLastError();
}

hipError_t launch_stream_read(const void* src, uint64_t bytes, hipStream_t stream) {
    const uint64_t pieces = bytes / 16384;
    const uint64_t blocks = (pieces + 7) / 8;
    const int grid = static_cast<int>(blocks < 1024 ? (blocks ? blocks : 1) : 1024);  // 4 workgroups per CU
    TraceScope trace("moe_stream_read", stream);
    stream_read_kernel<<<grid, 512, 0, stream>>>(static_cast<const u32x4*>(src), pieces);
    return hipGetLastError();
}

hipError_t launch_copy_bytes(void* dst, const void* src, uint64_t bytes, hipStream_t stream) {
    const uint64_t n16 = bytes / 16;
    const uint64_t blocks = (n16 + 255) / 256;
    const int grid = static_cast<int>(blocks < 8192 ? (blocks ? blocks : 1) : 8192);
    TraceScope trace("moe_copy_bytes", stream);
    copy_kernel<<<grid, 256, 0, stream>>>(static_cast<u32x4*>(dst), static_cast<const u32x4*>(src), n16);
    return hipGetLastError();
}

}  // namespace moe
