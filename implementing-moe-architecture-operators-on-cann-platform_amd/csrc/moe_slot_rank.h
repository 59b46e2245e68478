// moe_slot_rank.h -- stable ranking of a workgroup's range of (token, k) slots by expert id, on the device.
//
// Shared by the permute's count kernel (chunks of 1024 slots) and the routing kernels' optional tail (the
// slots of the token block a routing workgroup has just routed). The slot order is the oracle's
// (tests/moe_cpu_sim.cpp:412-418): for each expert, slots s = t*K + k ascending.
#pragma once

#include "moe_device.h"

namespace moe {

// Ranks the slots [s0, s1) by expert id (ids in [0, E), E <= 256; any other id belongs to no expert) with the
// workgroup's W waves. Wave w takes the R consecutive slots from s0 + w R (R = 64 ceil((s1 - s0) / (64 W)),
// at most 64 MAXIT), 64 at a time in slot order: lanes holding the same id find each other with 8 ballots over
// the id's bits, so a slot's rank among the wave's earlier slots of its expert is a popcount, and one lane per
// expert advances the wave's running count in LDS. Then rank[s] = the expert's slots in earlier waves + that
// wave-local rank, and counts_row[e] = the expert's slots in [s0, s1) for e < Ec (zeros for E <= e < Ec).
// wcnt: LDS scratch of W * E ints. Every thread of the workgroup calls this; it ends with a barrier.
template <int W, int MAXIT>
__device__ __forceinline__ void rank_slots(const int32_t* __restrict__ ids, int s0, int s1, int E, int Ec,
                                           int* wcnt, int32_t* __restrict__ counts_row,
                                           int32_t* __restrict__ rank) {
    const int tid = static_cast<int>(threadIdx.x);
    const int wave = __builtin_amdgcn_readfirstlane(tid / kWave);
    const int lane = lane_id();
    for (int i = tid; i < W * E; i += W * kWave) wcnt[i] = 0;
    __syncthreads();
    const int R = (s1 - s0 + kWave * W - 1) / (kWave * W) * kWave;
    const int b0 = s0 + wave * R, b1 = min(s1, b0 + R);
    const uint64_t below = (uint64_t{1} << lane) - 1;
    int e[MAXIT], r[MAXIT];
#pragma unroll
    for (int it = 0; it < MAXIT; ++it) {
        const int s = b0 + it * kWave + lane;
        e[it] = s < b1 ? ids[s] : -1;
    }
#pragma unroll
    for (int it = 0; it < MAXIT; ++it) {
        r[it] = 0;
        if (b0 + it * kWave >= b1) continue;  // uniform: this wave's range has ended
        const bool valid = e[it] >= 0 && e[it] < E;
        uint64_t same = __ballot(valid);  // lanes with a valid id equal to this lane's
#pragma unroll
        for (int b = 0; b < 8; ++b) {
            const bool bit = (e[it] >> b) & 1;
            const uint64_t m = __ballot(bit);
            same &= bit ? m : ~m;
        }
        const int before = __popcll(same & below);
        if (valid) {
            r[it] = wcnt[wave * E + e[it]] + before;
            // the lane of each expert's first slot advances the count; every lane's read above is issued first
            if (before == 0) wcnt[wave * E + e[it]] += __popcll(same);
        }
    }
    __syncthreads();
#pragma unroll
    for (int it = 0; it < MAXIT; ++it) {
        const int s = b0 + it * kWave + lane;
        if (s >= b1 || e[it] < 0 || e[it] >= E) continue;
        int prior = 0;  // the expert's slots in the earlier waves' ranges
        for (int w = 0; w < wave; ++w) prior += wcnt[w * E + e[it]];
        rank[s] = prior + r[it];
    }
    for (int x = tid; x < Ec; x += W * kWave) {
        int c = 0;
        if (x < E) {
#pragma unroll
            for (int w = 0; w < W; ++w) c += wcnt[w * E + x];
        }
        counts_row[x] = c;
    }
    __syncthreads();
}

// Row stride of the per-chunk expert counts: E rounded up to 4, so that each row is whole 16-byte quads.
__host__ __device__ constexpr int counts_stride(int E) { return (E + 3) / 4 * 4; }

}  // namespace moe
