// moe_slot_rank.h -- stable ranking of a workgroup's range of (token, k) slots by expert id, on the device.
//
// Shared by the permute's count kernel (chunks of 1024 slots) and the routing kernels' optional tail (the
// slots of the token block a routing workgroup has just routed). The slot order is the oracle's
// (tests/moe_cpu_sim.cpp:412-418): for each expert, slots s = t*K + k ascending.
#pragma once

#include "moe_device.h"

namespace moe {

// Ranks the slots [s0, s1) by expert id (ids in [0, E), E <= 256; any other id belongs to no expert) with the
// workgroup's W waves, in passes of up to W * 64 * MAXIT consecutive slots. In a pass wave w takes the R
// consecutive slots from the pass start + w R (R = 64 ceil(pass slots / (64 W))), 64 at a time in slot order:
// lanes holding the same id find each other with 8 ballots over the id's bits, so a slot's rank among the wave's
// earlier slots of its expert is a popcount, and one lane per expert advances the wave's running count in LDS.
// rank[s] = the expert's slots in earlier passes + in the pass's earlier waves + that wave-local rank, and
// counts_row[e] = the expert's slots in [s0, s1) for e < Ec (zeros for E <= e < Ec).
// wcnt: LDS scratch of (W + 1) * E ints. Every thread of the workgroup calls this; it ends with a barrier.
template <int W, int MAXIT>
__device__ __forceinline__ void rank_slots(const int32_t* __restrict__ ids, int s0, int s1, int E, int Ec,
                                           int* wcnt, int32_t* __restrict__ counts_row,
                                           int32_t* __restrict__ rank) {
    const int tid = static_cast<int>(threadIdx.x);
    const int wave = __builtin_amdgcn_readfirstlane(tid / kWave);
    const int lane = lane_id();
    int* base = wcnt + W * E;  // the experts' slots in earlier passes
    for (int i = tid; i < E; i += W * kWave) base[i] = 0;
    const uint64_t below = (uint64_t{1} << lane) - 1;
    constexpr int kSpan = W * kWave * MAXIT;
    for (int p0 = s0; p0 < s1; p0 += kSpan) {
        const int p1 = min(s1, p0 + kSpan);
        for (int i = tid; i < W * E; i += W * kWave) wcnt[i] = 0;
        __syncthreads();
        const int R = (p1 - p0 + kWave * W - 1) / (kWave * W) * kWave;
        const int b0 = p0 + wave * R, b1 = min(p1, b0 + R);
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
            int prior = base[e[it]];  // earlier passes, then the expert's slots in this pass's earlier waves
            for (int w = 0; w < wave; ++w) prior += wcnt[w * E + e[it]];
            rank[s] = prior + r[it];
        }
        __syncthreads();  // every rank is out before the pass's counts move into base
        for (int x = tid; x < E; x += W * kWave) {
            int c = 0;
#pragma unroll
            for (int w = 0; w < W; ++w) c += wcnt[w * E + x];
            base[x] += c;
        }
        __syncthreads();  // base is complete before the next pass clears wcnt, or before the counts go out
    }
    for (int x = tid; x < Ec; x += W * kWave) counts_row[x] = x < E ? base[x] : 0;
    __syncthreads();
}

// Row stride of the per-chunk expert counts: E rounded up to 4, so that each row is whole 16-byte quads.
__host__ __device__ constexpr int counts_stride(int E) { return (E + 3) / 4 * 4; }

}  // namespace moe
