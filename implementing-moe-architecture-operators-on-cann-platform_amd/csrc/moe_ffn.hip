// moe_ffn.hip -- MoeExpertFFN grouped GEMMs for gfx950.
//
// Reference: op_kernel/moe_expert_ffn.cpp (ComputeSwiGLU :265-333, ComputeDownProj :339-394, scatter
// :250-257) and the oracle's expert FFN, tests/moe_cpu_sim.cpp:245-296 (W_down read as [H, I]).
//
// Rows are the expert-sorted slots made by moe_permute.hip: expert e owns sorted rows
// [offsets[e], offsets[e+1]); sorted row r is slot sorted_slot[r] = t*K + k and its token is t.
//
// Weight-streaming schedule (few rows per expert, e.g. T = 128 decode): every weight byte is read from HBM
// once, so the layer is bound by streaming E*3*I*H*2 bytes.
//   gate/up kernel: one wave owns 16 intermediate rows i of one expert and walks the full hidden dim H:
//       per 32-wide k-step it loads the W_gate and W_up fragments (16 B per lane each, non-temporal) and
//       the token fragments of all row tiles of the expert (L2-resident), and issues two MFMAs per row tile.
//       Epilogue in registers: hidden = silu(gate) * up in fp32 -> fp16 into the workspace.
//   down kernel: one wave owns 16 hidden rows h of one expert's W_down [H, I], walks the full I dim, and
//       writes expert_out[slot, h] (fp16) directly for each sorted row -- the scatter is the epilogue.
// Both GEMMs are "NT": the weight rows and the activation rows are contiguous along the reduction dim,
// which is the 8-consecutive-k-per-lane operand format of v_mfma_f32_16x16x32_f16.
// Rows of an expert are processed in passes of up to 64 (4 MFMA row tiles); an expert with more rows
// re-streams its weights once per pass.

#include "moe_device.h"
#include "moe_launch.h"

namespace moe {

namespace {

constexpr int kWavesPerBlock = 4;

__device__ __forceinline__ float silu_f32(float g) { return g / (1.0f + expf(-g)); }

// One pass over `MT` 16-row tiles starting at expert-local row mc.
template <int MT>
__device__ __forceinline__ void gateup_pass(const uint16_t* __restrict__ x, const int32_t* __restrict__ sorted_slot,
                                            int off, int ne, int mc, int K, int H, int I,
                                            const uint16_t* __restrict__ wg, const uint16_t* __restrict__ wu,
                                            uint16_t* __restrict__ hidden, int n0, int lane) {
    const int row = lane & 15, kg = lane >> 4;
    const uint16_t* ap[MT];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
        const int r = min(mc + mt * 16 + row, ne - 1);  // padding rows reuse a valid row; results dropped
        const int slot = sorted_slot[off + r];
        ap[mt] = x + static_cast<size_t>(slot / K) * H + kg * 8;
    }
    f32x4 ag[MT], au[MT];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
        ag[mt] = f32x4{0.f, 0.f, 0.f, 0.f};
        au[mt] = f32x4{0.f, 0.f, 0.f, 0.f};
    }
#pragma unroll 4
    for (int k0 = 0; k0 < H; k0 += 32) {
        const f16x8 bg = load_f16x8_stream(wg + k0);
        const f16x8 bu = load_f16x8_stream(wu + k0);
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) {
            const f16x8 a = load_f16x8(ap[mt] + k0);
            ag[mt] = mfma16x16x32(a, bg, ag[mt]);
            au[mt] = mfma16x16x32(a, bu, au[mt]);
        }
    }
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int m = mc + mt * 16 + kg * 4 + r;
            if (m < ne) {
                const float hv = silu_f32(ag[mt][r]) * au[mt][r];
                hidden[static_cast<size_t>(off + m) * I + n0 + row] = f32_to_f16_bits(hv);
            }
        }
}

__global__ __launch_bounds__(kWavesPerBlock * kWave) void ffn_gateup_stream_kernel(
    const uint16_t* __restrict__ x, const int32_t* __restrict__ sorted_slot, const int32_t* __restrict__ offsets,
    const uint16_t* __restrict__ w, uint16_t* __restrict__ hidden, int E, int K, int H, int I) {
    const int lane = lane_id();
    const int gw = static_cast<int>(blockIdx.x) * kWavesPerBlock + static_cast<int>(threadIdx.x) / kWave;
    const int nb_per_expert = I / 16;
    if (gw >= E * nb_per_expert) return;
    const int e = gw / nb_per_expert;
    const int n0 = (gw % nb_per_expert) * 16;
    const int off = offsets[e];
    const int ne = offsets[e + 1] - off;
    if (ne <= 0) return;
    const int row = lane & 15, kg = lane >> 4;
    const size_t ebase = static_cast<size_t>(e) * 3 * static_cast<size_t>(I) * H;
    const uint16_t* wg = w + ebase + static_cast<size_t>(n0 + row) * H + kg * 8;
    const uint16_t* wu = wg + static_cast<size_t>(I) * H;
    int mc = 0;
    while (ne - mc > 32) {
        gateup_pass<4>(x, sorted_slot, off, ne, mc, K, H, I, wg, wu, hidden, n0, lane);
        mc += 64;
    }
    if (ne - mc > 16)
        gateup_pass<2>(x, sorted_slot, off, ne, mc, K, H, I, wg, wu, hidden, n0, lane);
    else if (ne - mc > 0)
        gateup_pass<1>(x, sorted_slot, off, ne, mc, K, H, I, wg, wu, hidden, n0, lane);
}

template <int MT>
__device__ __forceinline__ void down_pass(const uint16_t* __restrict__ hidden, const int32_t* __restrict__ sorted_slot,
                                          int off, int ne, int mc, int H, int I, const uint16_t* __restrict__ wd,
                                          uint16_t* __restrict__ expert_out, int n0, int lane) {
    const int row = lane & 15, kg = lane >> 4;
    const uint16_t* ap[MT];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
        const int r = min(mc + mt * 16 + row, ne - 1);
        ap[mt] = hidden + static_cast<size_t>(off + r) * I + kg * 8;
    }
    f32x4 acc[MT];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) acc[mt] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll 4
    for (int k0 = 0; k0 < I; k0 += 32) {
        const f16x8 b = load_f16x8_stream(wd + k0);
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) acc[mt] = mfma16x16x32(load_f16x8(ap[mt] + k0), b, acc[mt]);
    }
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int m = mc + mt * 16 + kg * 4 + r;
            if (m < ne) {
                const int slot = sorted_slot[off + m];
                expert_out[static_cast<size_t>(slot) * H + n0 + row] = f32_to_f16_bits(acc[mt][r]);
            }
        }
}

__global__ __launch_bounds__(kWavesPerBlock * kWave) void ffn_down_stream_kernel(
    const uint16_t* __restrict__ hidden, const int32_t* __restrict__ sorted_slot,
    const int32_t* __restrict__ offsets, const uint16_t* __restrict__ w, uint16_t* __restrict__ expert_out, int E,
    int H, int I) {
    const int lane = lane_id();
    const int gw = static_cast<int>(blockIdx.x) * kWavesPerBlock + static_cast<int>(threadIdx.x) / kWave;
    const int nb_per_expert = H / 16;
    if (gw >= E * nb_per_expert) return;
    const int e = gw / nb_per_expert;
    const int n0 = (gw % nb_per_expert) * 16;
    const int off = offsets[e];
    const int ne = offsets[e + 1] - off;
    if (ne <= 0) return;
    const int row = lane & 15, kg = lane >> 4;
    const size_t ebase = static_cast<size_t>(e) * 3 * static_cast<size_t>(I) * H;
    const uint16_t* wd = w + ebase + 2 * static_cast<size_t>(I) * H + static_cast<size_t>(n0 + row) * I + kg * 8;
    int mc = 0;
    while (ne - mc > 32) {
        down_pass<4>(hidden, sorted_slot, off, ne, mc, H, I, wd, expert_out, n0, lane);
        mc += 64;
    }
    if (ne - mc > 16)
        down_pass<2>(hidden, sorted_slot, off, ne, mc, H, I, wd, expert_out, n0, lane);
    else if (ne - mc > 0)
        down_pass<1>(hidden, sorted_slot, off, ne, mc, H, I, wd, expert_out, n0, lane);
}

size_t align_up(size_t v, size_t a) { return (v + a - 1) / a * a; }

}  // namespace

size_t ffn_workspace_bytes(int64_t T, int64_t E, int64_t K, int64_t I) {
    const size_t S = static_cast<size_t>(T) * static_cast<size_t>(K);
    size_t bytes = align_up(sizeof(int32_t) * static_cast<size_t>(E + 1), 256);
    bytes += align_up(sizeof(int32_t) * S, 256);
    bytes += align_up(sizeof(uint16_t) * S * static_cast<size_t>(I), 256);
    return bytes;
}

FfnWorkspace ffn_workspace_carve(void* base, int64_t T, int64_t E, int64_t K, int64_t I) {
    (void)I;
    const size_t S = static_cast<size_t>(T) * static_cast<size_t>(K);
    char* p = static_cast<char*>(base);
    FfnWorkspace ws;
    ws.offsets = reinterpret_cast<int32_t*>(p);
    p += align_up(sizeof(int32_t) * static_cast<size_t>(E + 1), 256);
    ws.sorted_slot = reinterpret_cast<int32_t*>(p);
    p += align_up(sizeof(int32_t) * S, 256);
    ws.hidden = reinterpret_cast<uint16_t*>(p);
    return ws;
}

FfnGrid ffn_grid(int T, int H, int E, int K, int I) {
    (void)T;
    (void)K;
    FfnGrid g;
    g.block_threads = kWavesPerBlock * kWave;
    g.gateup_blocks = (E * (I / 16) + kWavesPerBlock - 1) / kWavesPerBlock;
    g.down_blocks = (E * (H / 16) + kWavesPerBlock - 1) / kWavesPerBlock;
    g.rows_per_tile = 16;
    g.schedule = 0;
    return g;
}

hipError_t launch_ffn(const uint16_t* x, const uint16_t* expert_weights, uint16_t* expert_out, FfnWorkspace ws,
                      int T, int H, int E, int K, int I, hipStream_t stream) {
    const FfnGrid g = ffn_grid(T, H, E, K, I);
    {
        TraceScope trace("moe_ffn_gateup_swiglu", stream);
        ffn_gateup_stream_kernel<<<g.gateup_blocks, g.block_threads, 0, stream>>>(
            x, ws.sorted_slot, ws.offsets, expert_weights, ws.hidden, E, K, H, I);
    }
    hipError_t err = hipGetLastError();
    if (err != hipSuccess) return err;
    {
        TraceScope trace("moe_ffn_down", stream);
        ffn_down_stream_kernel<<<g.down_blocks, g.block_threads, 0, stream>>>(ws.hidden, ws.sorted_slot, ws.offsets,
                                                                               expert_weights, expert_out, E, H, I);
    }
    return hipGetLastError();
}

}  // namespace moe
