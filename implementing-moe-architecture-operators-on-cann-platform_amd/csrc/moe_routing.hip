// moe_routing.hip -- MoeRoutingTopK for gfx950.
//
// Reference: op_kernel/moe_routing.cpp (ComputeGate :238-254, SoftmaxRows :263-298, TopKSelect :304-369) and
// the CPU oracle NaiveMoE steps 1-3, tests/moe_cpu_sim.cpp:198-243.
//
// One workgroup owns 16 TB tokens (TB = 1, 2 or 4 blocks of 16, as many as keep >= 256 workgroups); W waves (16
// when E <= 32, else 4, bounded by the LDS of the partials). Each w_gate fragment a wave loads (8 strided 2-byte
// loads per lane) is multiplied into all TB token blocks: at T = 16384, E = 64 (TB = 4) that cut the kernel from
// 80 to 51 us (events), at T = 8192, E = 16 (TB = 2) from 16.6 to 15.2 us.
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
// For E > 64 a wide variant runs instead: a workgroup owns 64 tokens and each of its 4 waves 16 of them over
// all of H, so no partials are folded. w_gate reaches the waves through LDS: 32-row chunks are read with
// coalesced loads (one row of E experts is contiguous) and written transposed, [expert][h], so a lane's
// B fragment (8 consecutive h of one expert) is one ds_read_b128 instead of 8 strided 2-byte global loads.
// A stage of 2-4 such chunks (64-128 h) is loaded into registers while the previous one is multiplied, two
// LDS buffers, one barrier per stage. Measured at T = 16384, H = 2048, K = 6: E = 256 takes 206 us here
// against 425 us in the narrow kernel; at E = 64 the narrow kernel is faster (58 against 62 us: the
// transposing 2-byte LDS stores cost about what the strided global loads do), so it keeps E <= 64.
// HBM traffic per launch: T*H*2 (x) + H*E*2 (w_gate, L2-resident after the first workgroups) + T*K*6 bytes.

#include "moe_device.h"
#include "moe_launch.h"

namespace moe {

namespace {

constexpr int kTokensPerBlock = 16;

// The narrow kernel runs E <= 64. The wave count fixes each token's summation order (wave w adds the k-steps
// w, w + W, ... and the partials are folded in wave order), so it does not depend on the token blocks: a token's
// ids and weights are the same whatever T is. 8 waves at E = 64, T = 16384 were 5 % faster (48.9 against 51.3 us)
// but would make the bits depend on T.
constexpr int waves_for(int eb, int /*tb*/) { return eb <= 2 ? 16 : 4; }
// k-steps whose loads are issued together (E <= 32 runs 1024 threads: 128 VGPRs per lane; E <= 64 256), for tb
// 16-token blocks per workgroup
constexpr int unroll_for(int eb, int tb) {
    return tb == 1 ? (eb == 1 ? 4 : eb == 2 ? 2 : 4) : eb == 1 ? (tb == 2 ? 4 : 2) : eb == 2 ? (tb == 2 ? 2 : 1) : 2;
}
// 16-token blocks per workgroup of the narrow kernel: each w_gate fragment a wave loads feeds tb of them. As many
// as keep the grid at >= 256 workgroups (one per CU).
int narrow_token_blocks(int T) { return T >= 16 * 4 * 256 ? 4 : T >= 16 * 2 * 256 ? 2 : 1; }
constexpr size_t narrow_lds_bytes(int eb, int tb) {
    return static_cast<size_t>(waves_for(eb, tb)) * 16 * tb * eb * 16 * sizeof(float);
}

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

// EB = number of 16-expert blocks held in registers (ceil(E / 16) rounded up to an instantiated size); TB = 16-token
// blocks per workgroup (every w_gate fragment a wave loads is multiplied into all TB of them).
template <int EB, int TB>
__global__ __launch_bounds__(waves_for(EB, TB) * kWave) void routing_topk_kernel(const uint16_t* __restrict__ x,
                                                                              const uint16_t* __restrict__ w_gate,
                                                                              int32_t* __restrict__ expert_ids,
                                                                              uint16_t* __restrict__ weights, int T,
                                                                              int H, int E, int K) {
    constexpr int W = waves_for(EB, TB);
    constexpr int U = unroll_for(EB, TB);
    constexpr int Epad = EB * 16;
    constexpr int NT = 16 * TB;  // tokens per workgroup
    extern __shared__ float part[];  // [W][NT tokens][Epad] fp32 partial logits; row (0, t) receives the fold
    const int lane = lane_id();
    const int wave = static_cast<int>(threadIdx.x) / kWave;
    const int row = lane & 15;  // A row (token) / B column (expert) owned by this lane
    const int kg = lane >> 4;   // k-group: 8 consecutive k of each 32-wide k-step
    const int t0 = static_cast<int>(blockIdx.x) * NT;

    // ---- phase 1: partial logits on MFMA ----
    const uint16_t* xrow[TB];
#pragma unroll
    for (int tb = 0; tb < TB; ++tb) {
        const int tok = min(t0 + tb * 16 + row, T - 1);  // rows past T read a valid row; their results are dropped
        xrow[tb] = x + static_cast<size_t>(tok) * H + kg * 8;
    }
    f32x4 acc[TB][EB];
#pragma unroll
    for (int tb = 0; tb < TB; ++tb)
#pragma unroll
        for (int b = 0; b < EB; ++b) acc[tb][b] = f32x4{0.f, 0.f, 0.f, 0.f};

    const int nsteps = H / 32;
    for (int s0 = wave; s0 < nsteps; s0 += U * W) {
        f16x8 a[U][TB];
        f16x8 bv[U][EB];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int s = s0 + u * W;
            const bool in = s < nsteps;
            const int k0 = (in ? s : 0) * 32;
#pragma unroll
            for (int tb = 0; tb < TB; ++tb) {
                a[u][tb] = load_f16x8(xrow[tb] + k0);
                if (!in) {  // a k-step past H contributes nothing, whatever x holds (0 * inf would be NaN)
#pragma unroll
                    for (int q = 0; q < 8; ++q) a[u][tb][q] = static_cast<f16>(0.0f);
                }
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
            for (int tb = 0; tb < TB; ++tb)
#pragma unroll
                for (int b = 0; b < EB; ++b) acc[tb][b] = mfma16x16x32(a[u][tb], bv[u][b], acc[tb][b]);
    }
    // D[token tb*16 + 4*kg + r][expert b*16 + row]
#pragma unroll
    for (int tb = 0; tb < TB; ++tb)
#pragma unroll
        for (int b = 0; b < EB; ++b)
#pragma unroll
            for (int r = 0; r < 4; ++r) part[(wave * NT + tb * 16 + kg * 4 + r) * Epad + b * 16 + row] = acc[tb][b][r];
    __syncthreads();

    // ---- fold: partial of wave 0 + wave 1 + ... in wave order, into the wave-0 rows ----
    for (int i = static_cast<int>(threadIdx.x); i < NT * Epad; i += W * kWave) {
        float v = part[i];
#pragma unroll
        for (int w = 1; w < W; ++w) v += part[w * NT * Epad + i];
        part[i] = v;
    }
    __syncthreads();

    // ---- phase 2: one lane per token ----
    if (threadIdx.x >= NT) return;
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
        select_registers<Epad>(L, part + (NT + t) * Epad, E, K, ids_out, w_out);  // K <= E <= Epad
    } else {
        select_lds(part + t * Epad, part + (NT + t) * Epad, E, K, ids_out, w_out);  // wave-1 rows are free now
    }
}

constexpr int kWideTokens = 64;  // tokens per workgroup of the wide kernel
constexpr int kWideWaves = 4;    // one 16-token MFMA row block each

// chunks of 32 h per stage (one memory round trip per stage), sized to ~64 registers of staged w_gate per lane
constexpr int wide_chunks(int eb) { return eb == 8 ? 4 : 2; }
constexpr int wide_pitch(int eb) { return wide_chunks(eb) * 32 + 8; }  // halfs per transposed row (16 B padding)

// EB in {8, 16}: expert blocks of 16 (E <= 16 * EB)
template <int EB>
__global__ __launch_bounds__(kWideWaves * kWave) void routing_wide_kernel(const uint16_t* __restrict__ x,
                                                                           const uint16_t* __restrict__ w_gate,
                                                                           int32_t* __restrict__ expert_ids,
                                                                           uint16_t* __restrict__ weights, int T,
                                                                           int H, int E, int K) {
    constexpr int Epad = EB * 16;
    constexpr int CH = wide_chunks(EB);
    constexpr int P = wide_pitch(EB);
    constexpr int kThreads = kWideWaves * kWave;
    constexpr int kPer = (CH * 32 * Epad + kThreads - 1) / kThreads;  // w_gate elements per thread per stage
    extern __shared__ __align__(16) uint16_t wt[];                   // [2][Epad][P] halfs, then logits
    float* logits = reinterpret_cast<float*>(wt + 2 * Epad * P);     // [64 tokens][Epad] fp32
    const int tid = static_cast<int>(threadIdx.x);
    const int lane = lane_id();
    const int wave = tid / kWave;
    const int row = lane & 15, kg = lane >> 4;
    const int t0 = static_cast<int>(blockIdx.x) * kWideTokens;
    const int tok = min(t0 + wave * 16 + row, T - 1);  // rows past T read a valid row; results are dropped
    const uint16_t* xrow = x + static_cast<size_t>(tok) * H + kg * 8;
    const int nchunks = H / 32;
    const int nstages = (nchunks + CH - 1) / CH;

    // stage s of w_gate: rows 32*CH*s .. +32*CH, element q -> (h = q / E, e = q % E), coalesced along e;
    // rows past H read as zero
    uint16_t wv[kPer];
    f16x8 xa[CH];
    auto load_stage = [&](int st) {
        const int h0 = st * CH * 32;
        const int n = min(CH * 32, H - h0) * E;
#pragma unroll
        for (int j = 0; j < kPer; ++j) {
            const int q = tid + j * kThreads;
            wv[j] = q < n ? w_gate[static_cast<size_t>(h0) * E + q] : uint16_t{0};
        }
#pragma unroll
        for (int c = 0; c < CH; ++c) {
            if (st * CH + c < nchunks) {
                xa[c] = load_f16x8(xrow + h0 + c * 32);
            } else {  // a chunk past H contributes nothing, whatever x holds (0 * inf would be NaN)
#pragma unroll
                for (int q = 0; q < 8; ++q) xa[c][q] = static_cast<f16>(0.0f);
            }
        }
    };
    auto store_stage = [&](int buf) {
        uint16_t* dst = wt + buf * Epad * P;
#pragma unroll
        for (int j = 0; j < kPer; ++j) {
            const int q = tid + j * kThreads;
            if (q < CH * 32 * E) dst[(q % E) * P + q / E] = wv[j];
        }
    };
    // experts E..Epad-1 of both buffers read as zero
    for (int i = tid; i < 2 * (Epad - E) * P; i += kThreads) {
        const int b = i / ((Epad - E) * P), r = i % ((Epad - E) * P);
        wt[b * Epad * P + E * P + r] = 0;
    }

    f32x4 acc[EB];
#pragma unroll
    for (int b = 0; b < EB; ++b) acc[b] = f32x4{0.f, 0.f, 0.f, 0.f};
    load_stage(0);
    store_stage(0);
    f16x8 a[CH];
#pragma unroll
    for (int c = 0; c < CH; ++c) a[c] = xa[c];
    __syncthreads();
    for (int st = 0; st < nstages; ++st) {
        const int buf = st & 1;
        if (st + 1 < nstages) load_stage(st + 1);
        const uint16_t* src = wt + buf * Epad * P + row * P + kg * 8;
#pragma unroll
        for (int c = 0; c < CH; ++c)
#pragma unroll
            for (int b = 0; b < EB; ++b) {
                const f16x8 bv = *reinterpret_cast<const f16x8*>(src + b * 16 * P + c * 32);
                acc[b] = mfma16x16x32(a[c], bv, acc[b]);
            }
        if (st + 1 < nstages) {
            store_stage(buf ^ 1);  // that buffer was last read in stage st - 1
#pragma unroll
            for (int c = 0; c < CH; ++c) a[c] = xa[c];
        }
        __syncthreads();
    }
    // D[token 4*kg + r][expert b*16 + row] of this wave's 16 tokens
#pragma unroll
    for (int b = 0; b < EB; ++b)
#pragma unroll
        for (int r = 0; r < 4; ++r) logits[(wave * 16 + kg * 4 + r) * Epad + b * 16 + row] = acc[b][r];
    __syncthreads();

    // ---- one lane per token (wave 0) ----
    if (tid >= kWideTokens || t0 + tid >= T) return;
    const int t = tid;
    int32_t* ids_out = expert_ids + static_cast<size_t>(t0 + t) * K;
    uint16_t* w_out = weights + static_cast<size_t>(t0 + t) * K;
    float* picked = reinterpret_cast<float*>(wt) + t * 32;  // the w_gate buffers are free now: 32 floats a token
    if constexpr (EB <= 4) {
        float L[Epad];
#pragma unroll
        for (int e = 0; e < Epad; e += 4) {
            const f32x4 v = *reinterpret_cast<const f32x4*>(logits + t * Epad + e);
#pragma unroll
            for (int j = 0; j < 4; ++j) L[e + j] = v[j];
        }
        select_registers<Epad>(L, picked, E, K, ids_out, w_out);
    } else {
        select_lds(logits + t * Epad, picked, E, K, ids_out, w_out);
    }
}

size_t wide_lds_bytes(int eb) {
    const int pitch = eb == 8 ? wide_pitch(8) : wide_pitch(16);
    return static_cast<size_t>(2) * eb * 16 * pitch * sizeof(uint16_t) +
           static_cast<size_t>(kWideTokens) * eb * 16 * sizeof(float);
}

template <int EB>
hipError_t launch_wide(const uint16_t* x, const uint16_t* w_gate, int32_t* ids, uint16_t* w, int T, int H, int E,
                       int K, hipStream_t stream) {
    const int grid = (T + kWideTokens - 1) / kWideTokens;
    const size_t lds = wide_lds_bytes(EB);
    const hipError_t attr = ensure_lds_limit(reinterpret_cast<const void*>(&routing_wide_kernel<EB>),
                                             static_cast<int>(lds));
    if (attr != hipSuccess) return attr;
    TraceScope trace("moe_routing_topk", stream);
    routing_wide_kernel<EB><<<grid, kWideWaves * kWave, lds, stream>>>(x, w_gate, ids, w, T, H, E, K);
    return hipGetLastError();
}

template <int EB, int TB>
hipError_t launch_narrow(const uint16_t* x, const uint16_t* w_gate, int32_t* ids, uint16_t* w, int T, int H, int E,
                         int K, hipStream_t stream) {
    const int grid = (T + 16 * TB - 1) / (16 * TB);
    const size_t lds = narrow_lds_bytes(EB, TB);
    const hipError_t attr = ensure_lds_limit(reinterpret_cast<const void*>(&routing_topk_kernel<EB, TB>),
                                             static_cast<int>(lds));
    if (attr != hipSuccess) return attr;
    TraceScope trace("moe_routing_topk", stream);
    routing_topk_kernel<EB, TB><<<grid, waves_for(EB, TB) * kWave, lds, stream>>>(x, w_gate, ids, w, T, H, E, K);
    return hipGetLastError();
}

template <int EB>
hipError_t launch_eb(const uint16_t* x, const uint16_t* w_gate, int32_t* ids, uint16_t* w, int T, int H, int E,
                     int K, hipStream_t stream) {
    switch (narrow_token_blocks(T)) {
        case 1: return launch_narrow<EB, 1>(x, w_gate, ids, w, T, H, E, K, stream);
        case 2: return launch_narrow<EB, 2>(x, w_gate, ids, w, T, H, E, K, stream);
        default: return launch_narrow<EB, 4>(x, w_gate, ids, w, T, H, E, K, stream);
    }
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

int routing_tokens_per_block(int T, int E) {
    return routing_expert_blocks(E) <= 4 ? kTokensPerBlock * narrow_token_blocks(T) : kWideTokens;
}
int routing_block_threads(int T, int E) {
    const int eb = routing_expert_blocks(E);
    return eb <= 4 ? waves_for(eb, narrow_token_blocks(T)) * kWave : kWideWaves * kWave;
}
int routing_lds_bytes(int T, int E) {
    const int eb = routing_expert_blocks(E);
    if (eb > 4) return static_cast<int>(wide_lds_bytes(eb));
    return static_cast<int>(narrow_lds_bytes(eb, narrow_token_blocks(T)));
}

hipError_t launch_routing_topk(const uint16_t* x, const uint16_t* w_gate, int32_t* ids, uint16_t* w, int T, int H,
                               int E, int K, hipStream_t stream) {
    switch (routing_expert_blocks(E)) {
        case 1: return launch_eb<1>(x, w_gate, ids, w, T, H, E, K, stream);
        case 2: return launch_eb<2>(x, w_gate, ids, w, T, H, E, K, stream);
        case 4: return launch_eb<4>(x, w_gate, ids, w, T, H, E, K, stream);
        case 8: return launch_wide<8>(x, w_gate, ids, w, T, H, E, K, stream);
        default: return launch_wide<16>(x, w_gate, ids, w, T, H, E, K, stream);
    }
}

}  // namespace moe
