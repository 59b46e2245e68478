// moe_ffn.hip -- MoeExpertFFN: workspace layout and schedule dispatch of the grouped GEMMs.
//
// Reference: op_kernel/moe_expert_ffn.cpp:613-621 (kernel entry), op_host/moe_ops.cpp:340-349 (workspace).
// The expert FFN runs as three kernels on one stream:
//   moe_permute.hip      expert-sorted slot order + per-expert offsets (workspace)
//   gate/up + SwiGLU     hidden[r, :] = silu(x_t W_gate_e^T) * (x_t W_up_e^T) for sorted row r = (t, k), fp16
//   down + scatter       expert_out[t, k, :] = hidden[r, :] W_down_e^T, fp16
// The grouped GEMMs have two schedules (moe_ffn_stream.hip: weight streaming for few rows per expert).

#include "moe_device.h"
#include "moe_launch.h"

namespace moe {

namespace {

size_t align_up(size_t v, size_t a) { return (v + a - 1) / a * a; }

}  // namespace

// Layout (each region 256-byte aligned): offsets [E+1] i32 | sorted_slot [T*K] i32 | hidden [T*K, I] fp16 |
// partial [nsplit, T*K, H] fp32 (only when the down projection is split over K).
size_t ffn_workspace_bytes(int64_t T, int64_t H, int64_t E, int64_t K, int64_t I) {
    const size_t S = static_cast<size_t>(T) * static_cast<size_t>(K);
    size_t bytes = align_up(sizeof(int32_t) * static_cast<size_t>(E + 1), 256);
    bytes += align_up(sizeof(int32_t) * S, 256);
    bytes += align_up(sizeof(uint16_t) * S * static_cast<size_t>(I), 256);
    bytes += align_up(stream_partial_bytes(static_cast<int>(T), static_cast<int>(H), static_cast<int>(K),
                                           static_cast<int>(I)), 256);
    return bytes;
}

FfnWorkspace ffn_workspace_carve(void* base, int64_t T, int64_t H, int64_t E, int64_t K, int64_t I) {
    (void)H;
    const size_t S = static_cast<size_t>(T) * static_cast<size_t>(K);
    char* p = static_cast<char*>(base);
    FfnWorkspace ws;
    ws.offsets = reinterpret_cast<int32_t*>(p);
    p += align_up(sizeof(int32_t) * static_cast<size_t>(E + 1), 256);
    ws.sorted_slot = reinterpret_cast<int32_t*>(p);
    p += align_up(sizeof(int32_t) * S, 256);
    ws.hidden = reinterpret_cast<uint16_t*>(p);
    p += align_up(sizeof(uint16_t) * S * static_cast<size_t>(I), 256);
    ws.partial = reinterpret_cast<float*>(p);
    return ws;
}

FfnGrid ffn_grid(int T, int H, int E, int K, int I) {
    (void)T;
    (void)K;
    FfnGrid g;
    g.schedule = 0;
    g.block_threads = stream_block_threads();
    g.gateup_blocks = stream_gateup_grid(E, H, I);
    g.down_blocks = stream_down_grid(E, H, I);
    g.rows_per_tile = stream_rows_per_pass();
    return g;
}

hipError_t launch_ffn(const uint16_t* x, const uint16_t* expert_weights, uint16_t* expert_out, FfnWorkspace ws,
                      int T, int H, int E, int K, int I, hipStream_t stream) {
    return launch_ffn_stream(x, expert_weights, expert_out, ws, T, H, E, K, I, stream);
}

}  // namespace moe
