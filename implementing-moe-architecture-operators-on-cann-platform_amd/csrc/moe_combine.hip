// moe_combine.hip -- MoeCombine for gfx950: y[t, :] = sum_k weights[t, k] * expert_out[t, k, :].
//
// Reference: op_kernel/moe_combine.cpp:80-111 (which accumulates in fp16) and the oracle's combine,
// tests/moe_cpu_sim.cpp:298-305 / 499-538 (fp32 accumulator from 0.0f, k ascending).
//
// Pure HBM streaming: each thread owns 8 consecutive hidden elements of one token, loads the K fp16 rows
// with 16-byte loads (consecutive threads -> consecutive 16-byte chunks), accumulates in fp32 and stores 16
// bytes of y. Contraction into FMA is disabled in this file so every product and sum is rounded exactly as
// the oracle rounds it: for the same fp16 inputs, y is bit-identical to the oracle's fp32 result rounded to
// fp16 (round-to-nearest-even).
// Algorithmic HBM bytes per launch: T*K*H*2 (expert_out) + T*K*2 (weights) + T*H*2 (y).

#include "moe_device.h"
#include "moe_launch.h"

#pragma clang fp contract(off)

namespace moe {

namespace {

constexpr int kCombineThreads = 256;
constexpr int kElems = 8;
constexpr int kBatch = 8;
// expert_out larger than the 256 MB Infinity Cache is read with the non-temporal hint: it streams from HBM once and
// would only evict. Measured: DeepSeek shape (403 MB) 90.5 -> 82 us; at prefill (67 MB, still in the cache after
// the down projection wrote it) the hint made it slower, 21 -> 23 us.
constexpr int64_t kStreamOutBytes = int64_t(256) << 20;

template <bool NT>
__global__ __launch_bounds__(kCombineThreads) void combine_kernel(const uint16_t* __restrict__ expert_out,
                                                                  const uint16_t* __restrict__ weights,
                                                                  uint16_t* __restrict__ y, int T, int H, int K) {
    const int vec_per_row = H / kElems;
    const int64_t idx = static_cast<int64_t>(blockIdx.x) * kCombineThreads + threadIdx.x;
    if (idx >= static_cast<int64_t>(T) * vec_per_row) return;
    const int t = static_cast<int>(idx / vec_per_row);
    const int c = static_cast<int>(idx % vec_per_row) * kElems;
    float acc[kElems];
#pragma unroll
    for (int j = 0; j < kElems; ++j) acc[j] = 0.0f;
    const uint16_t* wrow = weights + static_cast<size_t>(t) * K;
    const uint16_t* orow = expert_out + static_cast<size_t>(t) * K * H + c;
    // up to kBatch rows are loaded before they are accumulated (still in ascending k)
    for (int k0 = 0; k0 < K; k0 += kBatch) {
        f16x8 o[kBatch];
        float w[kBatch];
#pragma unroll
        for (int u = 0; u < kBatch; ++u) {
            if (k0 + u < K) {
                w[u] = f16_bits_to_f32(wrow[k0 + u]);
                o[u] = NT ? load_f16x8_stream(orow + static_cast<size_t>(k0 + u) * H)
                          : load_f16x8(orow + static_cast<size_t>(k0 + u) * H);
            }
        }
#pragma unroll
        for (int u = 0; u < kBatch; ++u) {
            if (k0 + u < K) {
#pragma unroll
                for (int j = 0; j < kElems; ++j) acc[j] = acc[j] + w[u] * static_cast<float>(o[u][j]);
            }
        }
    }
    f16x8 out;
#pragma unroll
    for (int j = 0; j < kElems; ++j) out[j] = static_cast<f16>(acc[j]);
    *reinterpret_cast<f16x8*>(y + static_cast<size_t>(t) * H + c) = out;
}

}  // namespace

int combine_block_threads() { return kCombineThreads; }
int combine_elems_per_thread() { return kElems; }
int combine_grid(int64_t T, int64_t H) {
    const int64_t work = T * (H / kElems);
    return static_cast<int>((work + kCombineThreads - 1) / kCombineThreads);
}

hipError_t launch_combine(const uint16_t* expert_out, const uint16_t* weights, uint16_t* y, int T, int H, int K,
                          hipStream_t stream) {
    TraceScope trace("moe_combine", stream);
    if (static_cast<int64_t>(T) * K * H * 2 > kStreamOutBytes)
        combine_kernel<true><<<combine_grid(T, H), kCombineThreads, 0, stream>>>(expert_out, weights, y, T, H, K);
    else
        combine_kernel<false><<<combine_grid(T, H), kCombineThreads, 0, stream>>>(expert_out, weights, y, T, H, K);
    return hipGetLastError();
}

}  // namespace moe
