// moe_routing.hip -- MoeRoutingTopK for gfx950.
//
// Reference: op_kernel/moe_routing.cpp (ComputeGate :238-254, SoftmaxRows :263-298, TopKSelect :304-369) and
// the CPU oracle NaiveMoE steps 1-3, tests/moe_cpu_sim.cpp:198-243.
//
// One workgroup owns 16 tokens; W waves (16 when E <= 32, else 4, bounded by the LDS of the partials).
//   Phase 1: logits[16, E] = x[16, H] @ w_gate[H, E] on MFMA (v_mfma_f32_16x16x32_f16, fp32 accumulation;
//            fp16 x fp16 products are exact in fp32). The H/32 k-steps are dealt round-robin to the W waves; a
//            wave issues the loads of U k-steps before their MFMAs (at decode, H = 2048 and W = 16: all of a
//            wave's loads in one round trip), keeps partial logits of every expert block in registers and parks
//            them in LDS.
//   Fold:    one thread per (token, expert) adds the W partials in wave order.
//   Phase 2: one lane per token runs softmax, top-K and renormalisation sequentially over the experts, in the
//            oracle's order of operations: max scan from -1e30, expf(l - max), ascending-expert sum, division by
//            the sum; K rounds of a strict '>' scan (lowest index wins an exact tie); wSum over the K picks in
//            rank order; p / wSum; fp16 round-to-nearest-even. For E <= 64 the lane holds its row in registers
//            (16-byte LDS reads), otherwise it works on its LDS row.
// HBM traffic per launch: T*H*2 (x) + H*E*2 (w_gate, L2-resident after the first workgroups) + T*K*6 bytes.

#include "moe_device.h"
#include "moe_launch.h"

namespace moe {

namespace {

constexpr int kTokensPerBlock = 16;

constexpr int waves_for(int eb) { return eb <= 2 ? 16 : 4; }
// k-steps whose loads are issued together: E <= 32 runs 1024 threads (128 VGPRs per lane), larger E 256
constexpr int unroll_for(int eb) { return eb == 1 ? 4 : eb == 2 ? 2 : eb == 4 ? 4 : 2; }

// softmax + top-K + renormalisation of one token's logits L[0..E) held in registers (Epad = EB * 16 >= E)
template <int Epad>
__device__ __forceinline__ void select_registers(float (&L)[Epad], float* picked, int E, int K, int32_t* ids_out,
                                                 uint16_t* w_out) {
    float mx = -1e30f;
#pragma unroll
    for (int e = 0; e < Epad; ++e)
        if (e < E && L[e] > mx) mx = L[e];
    float total = 0.0f;
#pragma unroll
    for (int e = 0; e < Epad; ++e) {
        if (e < E) {
            L[e] = expf(L[e] - mx);
            total += L[e];
        }
    }
#pragma unroll
    for (int e = 0; e < Epad; ++e) L[e] = e < E ? L[e] / total : -2.0f;  // padding never wins a pick
    float sel = 0.0f;
    for (int k = 0; k < K; ++k) {
        float best = -1.0f;
        int bi = 0;
#pragma unroll
        for (int e = 0; e < Epad; ++e) {
            if (L[e] > best) {
                best = L[e];
                bi = e;
            }
        }
#pragma unroll
        for (int e = 0; e < Epad; ++e)
            if (e == bi) L[e] = -2.0f;  // probabilities are >= 0, so a picked expert never wins again
        ids_out[k] = bi;
        picked[k] = best;
        sel += best;
    }
    for (int k = 0; k < K; ++k) w_out[k] = f32_to_f16_bits(picked[k] / sel);
}

// the same on the token's LDS row (any E)
__device__ __forceinline__ void select_lds(float* L, float* picked, int E, int K, int32_t* ids_out,
                                           uint16_t* w_out) {
    float mx = -1e30f;
    for (int e = 0; e < E; ++e)
        if (L[e] > mx) mx = L[e];
    float total = 0.0f;
    for (int e = 0; e < E; ++e) {
        const float p = expf(L[e] - mx);
        L[e] = p;
        total += p;
    }
    for (int e = 0; e < E; ++e) L[e] = L[e] / total;
    float sel = 0.0f;
    for (int k = 0; k < K; ++k) {
        float best = -1.0f;
        int bi = 0;
        for (int e = 0; e < E; ++e) {
            const float v = L[e];
            if (v > best) {
                best = v;
                bi = e;
            }
        }
        ids_out[k] = bi;
        picked[k] = best;
        sel += best;
        L[bi] = -2.0f;
    }
    for (int k = 0; k < K; ++k) w_out[k] = f32_to_f16_bits(picked[k] / sel);
}

// EB = number of 16-expert blocks held in registers (ceil(E / 16) rounded up to an instantiated size).
template <int EB>
__global__ __launch_bounds__(waves_for(EB) * kWave) void routing_topk_kernel(const uint16_t* __restrict__ x,
                                                                              const uint16_t* __restrict__ w_gate,
                                                                              int32_t* __restrict__ expert_ids,
                                                                              uint16_t* __restrict__ weights, int T,
                                                                              int H, int E, int K) {
    constexpr int W = waves_for(EB);
    constexpr int U = unroll_for(EB);
    constexpr int Epad = EB * 16;
    extern __shared__ float part[];  // [W][16 tokens][Epad] fp32 partial logits; row (0, t) receives the fold
    const int lane = lane_id();
    const int wave = static_cast<int>(threadIdx.x) / kWave;
    const int row = lane & 15;  // A row (token) / B column (expert) owned by this lane
    const int kg = lane >> 4;   // k-group: 8 consecutive k of each 32-wide k-step
    const int t0 = static_cast<int>(blockIdx.x) * kTokensPerBlock;

    // ---- phase 1: partial logits on MFMA ----
    const int tok = min(t0 + row, T - 1);  // rows past T read a valid row; their results are dropped
    const uint16_t* xrow = x + static_cast<size_t>(tok) * H + kg * 8;
    f32x4 acc[EB];
#pragma unroll
    for (int b = 0; b < EB; ++b) acc[b] = f32x4{0.f, 0.f, 0.f, 0.f};

    const int nsteps = H / 32;
    for (int s0 = wave; s0 < nsteps; s0 += U * W) {
        f16x8 a[U];
        f16x8 bv[U][EB];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int s = s0 + u * W;
            const bool in = s < nsteps;
            const int k0 = (in ? s : 0) * 32;
            a[u] = load_f16x8(xrow + k0);
            if (!in) {  // a k-step past H contributes nothing, whatever x holds (0 * inf would be NaN)
#pragma unroll
                for (int q = 0; q < 8; ++q) a[u][q] = static_cast<f16>(0.0f);
            }
            const uint16_t* wrow = w_gate + static_cast<size_t>(k0 + kg * 8) * E;
#pragma unroll
            for (int b = 0; b < EB; ++b) {
                const int e = b * 16 + row;
#pragma unroll
                for (int q = 0; q < 8; ++q)
                    bv[u][b][q] = (in && e < E) ? __builtin_bit_cast(f16, wrow[static_cast<size_t>(q) * E + e])
                                                : static_cast<f16>(0.0f);
            }
        }
#pragma unroll
        for (int u = 0; u < U; ++u)
#pragma unroll
            for (int b = 0; b < EB; ++b) acc[b] = mfma16x16x32(a[u], bv[u][b], acc[b]);
    }
    // D[token 4*kg + r][expert b*16 + row]
#pragma unroll
    for (int b = 0; b < EB; ++b)
#pragma unroll
        for (int r = 0; r < 4; ++r) part[(wave * 16 + kg * 4 + r) * Epad + b * 16 + row] = acc[b][r];
    __syncthreads();

    // ---- fold: partial of wave 0 + wave 1 + ... in wave order, into the wave-0 rows ----
    for (int i = static_cast<int>(threadIdx.x); i < 16 * Epad; i += W * kWave) {
        float v = part[i];
#pragma unroll
        for (int w = 1; w < W; ++w) v += part[w * 16 * Epad + i];
        part[i] = v;
    }
    __syncthreads();

    // ---- phase 2: one lane per token ----
    if (threadIdx.x >= kTokensPerBlock) return;
    const int t = static_cast<int>(threadIdx.x);
    if (t0 + t >= T) return;
    int32_t* ids_out = expert_ids + static_cast<size_t>(t0 + t) * K;
    uint16_t* w_out = weights + static_cast<size_t>(t0 + t) * K;
    if constexpr (EB <= 4) {
        float L[Epad];
#pragma unroll
        for (int e = 0; e < Epad; e += 4) {
            const f32x4 v = *reinterpret_cast<const f32x4*>(part + t * Epad + e);
#pragma unroll
            for (int j = 0; j < 4; ++j) L[e + j] = v[j];
        }
        select_registers<Epad>(L, part + (16 + t) * Epad, E, K, ids_out, w_out);  // K <= E <= Epad
    } else {
        select_lds(part + t * Epad, part + (16 + t) * Epad, E, K, ids_out, w_out);  // wave-1 rows are free now
    }
}

template <int EB>
hipError_t launch_eb(const uint16_t* x, const uint16_t* w_gate, int32_t* ids, uint16_t* w, int T, int H, int E,
                     int K, hipStream_t stream) {
    const int grid = (T + kTokensPerBlock - 1) / kTokensPerBlock;
    const size_t lds = static_cast<size_t>(waves_for(EB)) * 16 * EB * 16 * sizeof(float);
    TraceScope trace("moe_routing_topk", stream);
    routing_topk_kernel<EB><<<grid, waves_for(EB) * kWave, lds, stream>>>(x, w_gate, ids, w, T, H, E, K);
    return hipGetLastError();
}

}  // namespace

int routing_expert_blocks(int E) {
    const int eb = (E + 15) / 16;
    if (eb <= 1) return 1;
    if (eb <= 2) return 2;
    if (eb <= 4) return 4;
    if (eb <= 8) return 8;
    return 16;
}

int routing_tokens_per_block() { return kTokensPerBlock; }
int routing_block_threads(int E) { return waves_for(routing_expert_blocks(E)) * kWave; }
int routing_lds_bytes(int E) {
    const int eb = routing_expert_blocks(E);
    return waves_for(eb) * 16 * eb * 16 * static_cast<int>(sizeof(float));
}

hipError_t launch_routing_topk(const uint16_t* x, const uint16_t* w_gate, int32_t* ids, uint16_t* w, int T, int H,
                               int E, int K, hipStream_t stream) {
    switch (routing_expert_blocks(E)) {
        case 1: return launch_eb<1>(x, w_gate, ids, w, T, H, E, K, stream);
        case 2: return launch_eb<2>(x, w_gate, ids, w, T, H, E, K, stream);
        case 4: return launch_eb<4>(x, w_gate, ids, w, T, H, E, K, stream);
        case 8: return launch_eb<8>(x, w_gate, ids, w, T, H, E, K, stream);
        default: return launch_eb<16>(x, w_gate, ids, w, T, H, E, K, stream);
    }
}

}  // namespace moe
