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
// Each pass is a chain of dependent round trips (16 loads per lane each). When E <= 255 and the T*K ids fit
// the LDS as bytes, pass 1 also keeps them there and pass 2 (and the zeroing below) reads the LDS copy.
// No atomics and no cleared memory, so the result is deterministic and needs no memset before the call.
// Slots whose id is outside [0, E) belong to no expert; the workgroups write zeros into their expert_out rows,
// each over 1/E of the slots (one workgroup doing it alone was the kernel's critical path: 40 us at 98304 slots).

#include "moe_device.h"
#include "moe_launch.h"

namespace moe {

namespace {

constexpr int kPermuteWaves = 16;
constexpr int kUnroll = 16;
constexpr int kPermuteLdsMax = 160 * 1024 - 1024;  // byte cache of the ids (dynamic LDS), static arrays aside

template <bool CACHE>
__global__ __launch_bounds__(kPermuteWaves * kWave) void permute_kernel(const int32_t* __restrict__ ids, int S, int E,
                                                                          int H, int32_t* __restrict__ offsets,
                                                                          int32_t* __restrict__ sorted_slot,
                                                                          uint16_t* __restrict__ expert_out) {
    extern __shared__ uint8_t id_cache[];  // CACHE: id of slot s at [s], 255 for ids outside [0, E)
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
            const bool valid = id[u] >= 0 && id[u] < E;
            n_eq += __popcll(__ballot(id[u] == e));
            n_lt += __popcll(__ballot(valid && id[u] < e));
            const int s = base + u * kWave + lane;
            if (CACHE && s < end) id_cache[s] = static_cast<uint8_t>(valid ? id[u] : 255);
        }
    }
    if (lane == 0) {
        cnt_eq[wave] = n_eq;
        cnt_lt[wave] = n_lt;
    }
    __syncthreads();  // the counts, and (CACHE) the byte copy of every chunk; each wave rereads only its own

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
            if (CACHE) {
                const int c = s < end ? static_cast<int>(id_cache[s]) : 255;
                id[u] = c == 255 ? -1 : c;
            } else {
                id[u] = s < end ? ids[s] : -1;
            }
        }
#pragma unroll
        for (int u = 0; u < kUnroll; ++u) {
            const uint64_t m = __ballot(id[u] == e);
            if (id[u] == e) sorted_slot[pos + __popcll(m & below)] = base + u * kWave + lane;
            pos += __popcll(m);
        }
    }

    // zero the expert_out rows of ids outside [0, E): workgroup e takes slots [e * per, (e + 1) * per), read from
    // its byte copy (CACHE) or with kUnroll loads in flight per thread
    const int per = (S + E - 1) / E;
    const int s_beg = min(S, e * per), s_end = min(S, s_beg + per);
    for (int base = s_beg; base < s_end; base += kUnroll * kPermuteWaves * kWave) {
        int id[kUnroll];
#pragma unroll
        for (int u = 0; u < kUnroll; ++u) {
            const int sl = base + u * kPermuteWaves * kWave + static_cast<int>(threadIdx.x);
            if (CACHE) {
                const int c = sl < s_end ? static_cast<int>(id_cache[sl]) : 0;
                id[u] = c == 255 ? -1 : c;
            } else {
                id[u] = sl < s_end ? ids[sl] : 0;
            }
        }
#pragma unroll
        for (int u = 0; u < kUnroll; ++u) {
            if (id[u] >= 0 && id[u] < E) continue;
            const int sl = base + u * kPermuteWaves * kWave + static_cast<int>(threadIdx.x);
            u32x4* row = reinterpret_cast<u32x4*>(expert_out + static_cast<size_t>(sl) * H);
            for (int j = 0; j < H / 8; ++j) row[j] = u32x4{0u, 0u, 0u, 0u};
        }
    }
}

}  // namespace

int permute_block_threads() { return kPermuteWaves * kWave; }

hipError_t prepare_permute(int S, int E) {
    if (E <= 255 && S <= kPermuteLdsMax)
        return ensure_lds_limit(reinterpret_cast<const void*>(&permute_kernel<true>), kPermuteLdsMax);
    return hipSuccess;
}

hipError_t launch_permute(const int32_t* ids, int S, int E, int H, FfnWorkspace ws, uint16_t* expert_out,
                          hipStream_t stream) {
    TraceScope trace("moe_permute", stream);
    if (E <= 255 && S <= kPermuteLdsMax) {
        const void* fn = reinterpret_cast<const void*>(&permute_kernel<true>);
        const hipError_t attr = ensure_lds_limit(fn, kPermuteLdsMax);
        if (attr != hipSuccess) return attr;
        permute_kernel<true><<<E, kPermuteWaves * kWave, static_cast<size_t>(S), stream>>>(
            ids, S, E, H, ws.offsets, ws.sorted_slot, expert_out);
    } else {
        permute_kernel<false><<<E, kPermuteWaves * kWave, 0, stream>>>(ids, S, E, H, ws.offsets, ws.sorted_slot,
                                                                        expert_out);
    }
    return hipGetLastError();
}

}  // namespace moe
