// moe_permute.hip -- token permutation for MoeExpertFFN: expert-sorted slot order plus per-expert offsets.
//
// Reference: the per-expert scan of expert_ids in op_kernel/moe_expert_ffn.cpp:182-195 (capped at 512 rows)
// and, for the order, the oracle's (token, slot) collection in tests/moe_cpu_sim.cpp:412-418: for each expert,
// slots s = t*K + k in ascending order. Here there is no cap.
//
// One workgroup of 16 waves per expert e. The T*K ids are cut into 16 contiguous chunks, one per wave.
//   pass 1: each wave counts, with 64-lane ballots, the ids equal to e and the valid ids below e in its chunk;
//   the workgroup sums them: offsets[e] = #(valid ids < e), and each wave's first output row;
//   pass 2: each wave rescans its chunk and writes the slots of expert e in ascending order.
// No atomics and no cleared memory, so the result is deterministic and needs no memset before the call.
// Slots whose id is outside [0, E) belong to no expert; workgroup 0 writes zeros into their expert_out rows.

#include "moe_device.h"
#include "moe_launch.h"

namespace moe {

namespace {

constexpr int kPermuteWaves = 16;
constexpr int kUnroll = 8;

__global__ __launch_bounds__(kPermuteWaves * kWave) void permute_kernel(const int32_t* __restrict__ ids, int S, int E,
                                                                          int H, int32_t* __restrict__ offsets,
                                                                          int32_t* __restrict__ sorted_slot,
                                                                          uint16_t* __restrict__ expert_out) {
    __shared__ int cnt_eq[kPermuteWaves];
    __shared__ int cnt_lt[kPermuteWaves];
    const int e = static_cast<int>(blockIdx.x);
    const int lane = lane_id();
    const int wave = static_cast<int>(threadIdx.x) / kWave;
    const int chunk = (((S + kPermuteWaves - 1) / kPermuteWaves) + kWave - 1) / kWave * kWave;
    const int beg = min(S, wave * chunk);
    const int end = min(S, beg + chunk);

    // kUnroll loads per lane are issued before their ballots: the chunk is read in a few round trips
    int n_eq = 0, n_lt = 0;
    for (int base = beg; base < end; base += kUnroll * kWave) {
        int id[kUnroll];
#pragma unroll
        for (int u = 0; u < kUnroll; ++u) {
            const int s = base + u * kWave + lane;
            id[u] = s < end ? ids[s] : -1;
        }
#pragma unroll
        for (int u = 0; u < kUnroll; ++u) {
            n_eq += __popcll(__ballot(id[u] == e));
            n_lt += __popcll(__ballot(id[u] >= 0 && id[u] < e));
        }
    }
    if (lane == 0) {
        cnt_eq[wave] = n_eq;
        cnt_lt[wave] = n_lt;
    }
    __syncthreads();

    int off = 0, before = 0, total_eq = 0;
    for (int w = 0; w < kPermuteWaves; ++w) {
        off += cnt_lt[w];
        total_eq += cnt_eq[w];
        if (w < wave) before += cnt_eq[w];
    }
    if (threadIdx.x == 0) {
        offsets[e] = off;
        if (e == E - 1) offsets[E] = off + total_eq;
    }

    const uint64_t below = (uint64_t{1} << lane) - 1;
    int pos = off + before;
    for (int base = beg; base < end; base += kUnroll * kWave) {
        int id[kUnroll];
#pragma unroll
        for (int u = 0; u < kUnroll; ++u) {
            const int s = base + u * kWave + lane;
            id[u] = s < end ? ids[s] : -1;
        }
#pragma unroll
        for (int u = 0; u < kUnroll; ++u) {
            const uint64_t m = __ballot(id[u] == e);
            if (id[u] == e) sorted_slot[pos + __popcll(m & below)] = base + u * kWave + lane;
            pos += __popcll(m);
        }
    }

    if (e != 0) return;
    for (int s = static_cast<int>(threadIdx.x); s < S; s += kPermuteWaves * kWave) {
        const int id = ids[s];
        if (id >= 0 && id < E) continue;
        u32x4* row = reinterpret_cast<u32x4*>(expert_out + static_cast<size_t>(s) * H);
        for (int j = 0; j < H / 8; ++j) row[j] = u32x4{0u, 0u, 0u, 0u};
    }
}

}  // namespace

int permute_block_threads() { return kPermuteWaves * kWave; }

hipError_t launch_permute(const int32_t* ids, int S, int E, int H, FfnWorkspace ws, uint16_t* expert_out,
                          hipStream_t stream) {
    TraceScope trace("moe_permute", stream);
    permute_kernel<<<E, kPermuteWaves * kWave, 0, stream>>>(ids, S, E, H, ws.offsets, ws.sorted_slot, expert_out);
    return hipGetLastError();
}

}  // namespace moe
