// moe_permute.hip -- token permutation for MoeExpertFFN: expert-sorted slot order plus per-expert offsets.
//
// Reference: the per-expert scan of expert_ids in op_kernel/moe_expert_ffn.cpp:182-195 (capped at 512 rows)
// and, for the order, the oracle's (token, slot) collection in tests/moe_cpu_sim.cpp:412-418: for each expert,
// slots s = t*K + k in ascending order. Here there is no cap.
//
// A stable counting sort of the T*K slots by expert id over chunks of consecutive slots:
//   count    per chunk, each slot's rank among the chunk's earlier slots of its expert (rank[s]) and the chunk's
//            per-expert counts (counts[chunk][e], rows of counts_stride(E) ints): rank_slots, either in
//            permute_count_kernel (one workgroup per chunk of kChunk slots) or in the routing kernel's tail
//            (one chunk per routing workgroup: its token block's slots), which saves this launch.
//   scatter  one workgroup per cpw consecutive chunks sums the counts columns over all chunks (each expert's
//            total) and over the chunks before its own (16-byte loads of 4 experts, 16 in flight per thread);
//            its first slots' ids and ranks are loaded before those sums;
//            a scan over the experts gives offsets[e], a scan over its own chunks each chunk's base, and slot s
//            of expert e in chunk c goes to sorted_slot[offsets[e] + (e's slots in chunks before c) + rank[s]].
//            Workgroup 0 writes offsets.
// No atomics and no cleared memory, so the result is deterministic and needs no memset before the call.
// Slots whose id is outside [0, E) belong to no expert; the scatter workgroups write zeros into their expert_out
// rows, each over its own chunks.
// Replaces one workgroup per expert scanning all T*K ids (O(E*T*K) reads: 29.5 us at T*K = 98304, E = 64).

#include "moe_launch.h"
#include "moe_slot_rank.h"

namespace moe {

namespace {

constexpr int kThreads = 256;         // 4 waves
constexpr int kChunk = 4 * kThreads;  // slots per count workgroup: 256 per wave, 64 per step
constexpr int kMaxE = 256;            // the library's expert limit (8 id bits)
constexpr int kMaxCpw = 16;           // chunks per scatter workgroup
constexpr int kInFlight = 16;         // counts loads per thread in flight
constexpr int kScatterThreads = 256;  // 4 waves per scatter workgroup (1024 was slower)

__global__ __launch_bounds__(kThreads) void permute_count_kernel(const int32_t* __restrict__ ids, int S, int E,
                                                                 int32_t* __restrict__ counts,
                                                                 int32_t* __restrict__ rank) {
    __shared__ int wcnt[(kThreads / kWave + 1) * kMaxE];
    const int s0 = static_cast<int>(blockIdx.x) * kChunk;
    rank_slots<kThreads / kWave, 4>(ids, s0, min(S, s0 + kChunk), E, counts_stride(E), wcnt,
                                    counts + static_cast<size_t>(blockIdx.x) * counts_stride(E), rank);
}

__global__ __launch_bounds__(kScatterThreads) void permute_scatter_kernel(
    const int32_t* __restrict__ ids, int S, int E, int H, const int32_t* __restrict__ counts,
    const int32_t* __restrict__ rank, int nchunks, int chunk_slots, int cpw, int32_t* __restrict__ offsets,
    int32_t* __restrict__ sorted_slot, uint16_t* __restrict__ expert_out) {
    __shared__ int4 sum_tot[kScatterThreads], sum_pre[kScatterThreads];
    __shared__ int total_e[kMaxE], pre_e[kMaxE];
    __shared__ int lbase[kMaxCpw * kMaxE];  // [own chunk][expert]: counts, then each chunk's base
    __shared__ int wsum[kScatterThreads / kWave];
    const int tid = static_cast<int>(threadIdx.x);
    const int wave = tid / kWave, lane = lane_id();
    const int Ec = counts_stride(E);
    const int c0 = static_cast<int>(blockIdx.x) * cpw, c1 = min(nchunks, c0 + cpw);

    // the first slots of the scatter below: ids and ranks loaded now, under the column sums
    constexpr int kBatch = 8;
    const int s_begin = c0 * chunk_slots, s_end = min(S, c1 * chunk_slots);
    int e[kBatch], r[kBatch];
    auto load_batch = [&](int sb) __attribute__((always_inline)) {
#pragma unroll
        for (int u = 0; u < kBatch; ++u) {
            const int s = sb + u * kScatterThreads;
            e[u] = s < s_end ? ids[s] : 0;
            r[u] = s < s_end ? rank[s] : 0;
        }
    };
    load_batch(s_begin + tid);
    // this workgroup's own chunks' counts (they do not depend on the column sums)
    for (int i = tid; i < (c1 - c0) * E; i += kScatterThreads) {
        const int c = i / E, x = i % E;
        lbase[c * E + x] = counts[static_cast<size_t>(c0 + c) * Ec + x];
    }
    // column sums: thread t takes quad q = t % Q (experts 4q..4q+3) of the chunks p, p + P, ... (p = t / Q, P <= 64)
    const int Q = Ec / 4, P = min(64, kScatterThreads / Q);
    if (tid < P * Q) {
        const int q = tid % Q, p = tid / Q;
        int4 tot = {0, 0, 0, 0}, pre = {0, 0, 0, 0};
        for (int ch0 = p; ch0 < nchunks; ch0 += kInFlight * P) {
            int4 v[kInFlight];
#pragma unroll
            for (int u = 0; u < kInFlight; ++u) {
                const int ch = ch0 + u * P;
                v[u] = ch < nchunks ? *reinterpret_cast<const int4*>(counts + static_cast<size_t>(ch) * Ec + 4 * q)
                                    : int4{0, 0, 0, 0};
            }
#pragma unroll
            for (int u = 0; u < kInFlight; ++u) {
                tot.x += v[u].x; tot.y += v[u].y; tot.z += v[u].z; tot.w += v[u].w;
                if (ch0 + u * P < c0) {
                    pre.x += v[u].x; pre.y += v[u].y; pre.z += v[u].z; pre.w += v[u].w;
                }
            }
        }
        sum_tot[tid] = tot;
        sum_pre[tid] = pre;
    }
    __syncthreads();
    // per expert: 4 consecutive lanes (t = 4 x + j) add the parts p = j, j + 4, ..., then two xor shuffles; the
    // workgroup covers kScatterThreads / 4 experts per round
    for (int x0 = 0; x0 < E; x0 += kScatterThreads / 4) {
        const int x = x0 + tid / 4, j = tid % 4;
        int tot = 0, pre = 0;
        if (x < E) {
            const int q = x / 4, c = x % 4;
            for (int pp = j; pp < P; pp += 4) {
                const int4 a = sum_tot[pp * Q + q], b = sum_pre[pp * Q + q];
                tot += c == 0 ? a.x : c == 1 ? a.y : c == 2 ? a.z : a.w;
                pre += c == 0 ? b.x : c == 1 ? b.y : c == 2 ? b.z : b.w;
            }
        }
        tot += __shfl_xor(tot, 1, kWave);
        pre += __shfl_xor(pre, 1, kWave);
        tot += __shfl_xor(tot, 2, kWave);
        pre += __shfl_xor(pre, 2, kWave);
        if (x < E && j == 0) {
            total_e[x] = tot;
            pre_e[x] = pre;
        }
    }
    __syncthreads();
    const int total = tid < E ? total_e[tid] : 0;  // thread x < E: expert x
    // exclusive scan of the totals over the experts (one wave-level scan per wave, then the wave sums)
    int incl = total;
#pragma unroll
    for (int d = 1; d < kWave; d <<= 1) {
        const int v = __shfl_up(incl, d, kWave);
        if (lane >= d) incl += v;
    }
    if (lane == kWave - 1) wsum[wave] = incl;
    __syncthreads();
    int carry = 0;
    for (int w = 0; w < wave; ++w) carry += wsum[w];
    const int off = carry + incl - total;
    if (tid < E) {
        // each own chunk's base for this expert: offset + earlier chunks' slots of the expert
        int run = off + pre_e[tid];
        for (int c = 0; c < c1 - c0; ++c) {
            const int n = lbase[c * E + tid];
            lbase[c * E + tid] = run;
            run += n;
        }
        if (blockIdx.x == 0) offsets[tid] = off;
    }
    if (blockIdx.x == 0 && tid == E - 1) offsets[E] = off + total;
    __syncthreads();

    // the scatter, kBatch slots per thread at a time, their ids and ranks loaded before any store
    for (int sb = s_begin + tid; sb < s_end; sb += kBatch * kScatterThreads) {
        if (sb != s_begin + tid) load_batch(sb);
#pragma unroll
        for (int u = 0; u < kBatch; ++u) {
            const int s = sb + u * kScatterThreads;
            if (s >= s_end) continue;
            if (e[u] >= 0 && e[u] < E) {
                sorted_slot[lbase[(s / chunk_slots - c0) * E + e[u]] + r[u]] = s;
            } else {  // belongs to no expert: its expert_out row is zero
                u32x4* row = reinterpret_cast<u32x4*>(expert_out + static_cast<size_t>(s) * H);
                for (int jj = 0; jj < H / 8; ++jj) row[jj] = u32x4{0u, 0u, 0u, 0u};
            }
        }
    }
}

}  // namespace

int permute_block_threads() { return kThreads; }
int permute_chunks(int S) { return (S + kChunk - 1) / kChunk; }

// rank [S] i32, then (16-byte aligned) counts [chunks][counts_stride(E)] i32
size_t permute_scratch_bytes(int S, int E) {
    return static_cast<size_t>(counts_stride(S)) * sizeof(int32_t) +
           static_cast<size_t>(permute_chunks(S)) * counts_stride(E) * sizeof(int32_t);
}

hipError_t prepare_permute(int S, int E) {
    (void)S;
    (void)E;
    return hipSuccess;  // static LDS only
}

int permute_scatter_chunks_per_block(int nchunks) {
    // about 256 scatter workgroups (one per CU). T = 16384, E = 64, K = 6 (512 chunks of 192 slots): 2 chunks per
    // workgroup 8.1 us, 4: 8.3, 8: 8.8, 16: 11.3 (each workgroup then sums more count rows and scatters more)
    return min(kMaxCpw, max(1, (nchunks + 255) / 256));
}

hipError_t launch_permute_scatter(const int32_t* ids, int S, int E, int H, const int32_t* counts,
                                  const int32_t* rank, int nchunks, int chunk_slots, int cpw, FfnWorkspace ws,
                                  uint16_t* expert_out, hipStream_t stream) {
    if (cpw < 1 || cpw > kMaxCpw) return hipErrorInvalidValue;
    TraceScope trace("moe_permute_scatter", stream);
    permute_scatter_kernel<<<(nchunks + cpw - 1) / cpw, kScatterThreads, 0, stream>>>(
        ids, S, E, H, counts, rank, nchunks, chunk_slots, cpw, ws.offsets, ws.sorted_slot, expert_out);
    return hipGetLastError();
}

hipError_t launch_permute(const int32_t* ids, int S, int E, int H, FfnWorkspace ws, uint16_t* expert_out,
                          hipStream_t stream) {
    const int nchunks = permute_chunks(S);
    int32_t* rank = ws.pscratch;
    int32_t* counts = ws.pscratch + counts_stride(S);  // 16-byte aligned rows
    {
        TraceScope trace("moe_permute", stream);
        permute_count_kernel<<<nchunks, kThreads, 0, stream>>>(ids, S, E, counts, rank);
    }
    hipError_t err = hipGetLastError();
    if (err != hipSuccess) return err;
    return launch_permute_scatter(ids, S, E, H, counts, rank, nchunks, kChunk, 1, ws, expert_out, stream);
}

}  // namespace moe
