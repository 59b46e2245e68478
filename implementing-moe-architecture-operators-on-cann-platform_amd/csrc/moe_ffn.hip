// moe_ffn.hip -- MoeExpertFFN: workspace layout and schedule dispatch of the grouped GEMMs.
//
// Reference: op_kernel/moe_expert_ffn.cpp:613-621 (kernel entry), op_host/moe_ops.cpp:340-349 (workspace).
// The expert FFN runs on one stream as
//   permute              expert-sorted slot order + per-expert offsets (workspace): moe_permute.hip for the
//                        tiled schedule; the streaming gate/up kernel finds its rows itself
//   gate/up + SwiGLU     hidden[r, :] = silu(x_t W_gate_e^T) * (x_t W_up_e^T) for sorted row r = (t, k), fp16
//   down + scatter       expert_out[t, k, :] = hidden[r, :] W_down_e^T, fp16
// The grouped GEMMs have two schedules, chosen on the host from the average number of rows per expert
// (the actual per-expert counts exist only on the device):
//   moe_ffn_stream.hip  weight streaming, for few rows per expert (HBM-bound: every weight byte read once)
//   moe_ffn_tiled.hip   256x256 LDS-tiled MFMA tiles, for many rows per expert (MFMA-bound)

#include "moe_device.h"
#include "moe_launch.h"
#include "moe_slot_rank.h"

namespace moe {

namespace {

size_t align_up(size_t v, size_t a) { return (v + a - 1) / a * a; }

// Average rows per expert from which the tiled schedule runs. The 32-row streaming kernels stream every expert's
// weights once per 32 rows, so they degrade once experts exceed 32 rows; the wide streaming kernels take up to 128
// rows per pass and run in their place from 32 rows (moe_ffn_stream.hip); the tiled kernels cost about the same
// from 32 to 256 rows (their 256-row tiles are then mostly padding). H = 2048, E = 16, K = 2, I = 8192, the FFN's
// kernels on one box (32-row streaming / wide streaming / tiled):
//   T = 128 (16 rows per expert)   273 / -   / 466 us
//   T = 256 (32)                    451 / 364 / 449-493 us
//   T = 384 (48)                    541 / 385 / 458-491 us
//   T = 512 (64)                    707 / 440 / 452-477 us
//   T = 768 (96)                      - / 496 / 465-482 us
//   T = 1024 (128)                 1271 / 734 / 480-491 us
// The wide/tiled crossover moves with I: the FFN (wide / tiled, us) at 64 and 80 rows per expert on average:
//   H = 2048, E = 16, K = 2, I = 8192     420 / 501,  445 / 496   (wide still ahead at 80 rows)
//   H = 4096, E = 8,  K = 2, I = 14336    676 / 816,  765 / 843
//   H = 2048, E = 64, K = 6, I = 1408     332 / 353,  350 / 333   (crossover ~72 rows)
//   H = 4096, E = 128, K = 8, I = 1536   1160 / 1241, 1264 / 1250  (~77)
//   H = 5120, E = 16, K = 2, I = 1536     241 / 253,  270 / 264   (~74)
//   H = 7168, E = 256, K = 8, I = 2048   5427 / 5297 at 64 rows, 5029 / 5259 at 56  (~61)
// so the wide kernels run to 72 rows below I = 4096. From I = 4096 they run to 96 rows, measured again with the
// wide kernels' short passes (moe_ffn_stream.hip), the FFN (wide / tiled, us, one box):
//   H = 2048, E = 16, K = 2, I = 8192     80 rows 408.6 / 442.2, 88 rows 419.6 / 452.4, 96 rows 431.8 / 450.8,
//                                         112 rows 612.5 / 468.1 (experts above 128 rows take a second pass)
//   H = 4096, E = 8,  K = 2, I = 14336    80 rows 726.7 / 784.0, 96 rows 779.1 / 804.8, 112 rows 1143.3 / 822.5
// Shapes the wide kernels cannot run switch to the tiled schedule at 32 rows.
constexpr int64_t kTiledMinRowsPerExpert = 32;
constexpr int64_t kWideMaxRowsPerExpert = 97;
constexpr int64_t kWideMaxRowsSmallI = 72;
constexpr int64_t kWideLargeI = 4096;

}  // namespace

int ffn_schedule(int64_t T, int64_t H, int64_t E, int64_t K, int64_t I, FfnSplits splits) {
    const bool stream_ok = stream_supported(static_cast<int>(H), static_cast<int>(I), splits.gateup);
    const int64_t wide_limit = I >= kWideLargeI ? kWideMaxRowsPerExpert : kWideMaxRowsSmallI;
    const int64_t limit = stream_wide_supported(static_cast<int>(H), static_cast<int>(I)) ? wide_limit
                                                                                          : kTiledMinRowsPerExpert;
    const bool many_rows = T * K >= limit * E;
    if (tiled_shape_supported(H, E, I) && (many_rows || !stream_ok))
        return tiled_size_supported(T, H, K, I) ? 1 : -1;
    if (stream_ok) return 0;
    return -1;
}

// Layout (each region 256-byte aligned): offsets [E+1] i32 | sorted_slot [T*K] i32 | hidden [T*K, I] fp16, then
// for the weight-streaming schedule: fp32 partial sums, [nsplit, T*K, H] when the down projection is split over K
// and [nsplit, T*K, 2*I] when the 32-row gate/up kernel splits H (the larger of the two; one serves both in turn) |
// slot_row [T*K] i32; for the tiled schedule: the permute's scratch (rank [T*K] i32, counts [chunks, E] i32),
// then with splits.tiled up to 256 fp32 partial tiles of 256 x 256 (64 MiB; one per workgroup of the down launch)
// for the leftover round it splits over k (none when I < 256 or when the down tiles fill more than 4 rounds).
size_t ffn_workspace_bytes(int64_t T, int64_t H, int64_t E, int64_t K, int64_t I, FfnSplits splits) {
    const size_t S = static_cast<size_t>(T) * static_cast<size_t>(K);
    size_t bytes = align_up(sizeof(int32_t) * static_cast<size_t>(E + 1), 256);
    bytes += align_up(sizeof(int32_t) * S, 256);
    bytes += align_up(sizeof(uint16_t) * S * static_cast<size_t>(I), 256);
    const int schedule = ffn_schedule(T, H, E, K, I, splits);
    if (schedule == 0) {
        bytes += align_up(stream_partial_bytes(static_cast<int>(T), static_cast<int>(H), static_cast<int>(E),
                                               static_cast<int>(K), static_cast<int>(I), stream_wide(T, H, E, K, I),
                                               splits.gateup), 256);
        bytes += align_up(sizeof(int32_t) * S, 256);
    } else if (schedule == 1) {
        bytes += align_up(permute_scratch_bytes(static_cast<int>(S), static_cast<int>(E)), 256);
        if (splits.tiled)
            bytes += align_up(tiled_partial_bytes(static_cast<int>(T), static_cast<int>(H), static_cast<int>(E),
                                                  static_cast<int>(K), static_cast<int>(I)), 256);
    }
    return bytes;
}

FfnWorkspace ffn_workspace_carve(void* base, int64_t T, int64_t H, int64_t E, int64_t K, int64_t I,
                                 FfnSplits splits) {
    const size_t S = static_cast<size_t>(T) * static_cast<size_t>(K);
    char* p = static_cast<char*>(base);
    FfnWorkspace ws;
    ws.offsets = reinterpret_cast<int32_t*>(p);
    p += align_up(sizeof(int32_t) * static_cast<size_t>(E + 1), 256);
    ws.sorted_slot = reinterpret_cast<int32_t*>(p);
    p += align_up(sizeof(int32_t) * S, 256);
    ws.hidden = reinterpret_cast<uint16_t*>(p);
    p += align_up(sizeof(uint16_t) * S * static_cast<size_t>(I), 256);
    ws.partial = nullptr;
    ws.slot_row = nullptr;
    ws.pscratch = nullptr;
    const int schedule = ffn_schedule(T, H, E, K, I, splits);
    if (schedule == 0) {
        ws.partial = reinterpret_cast<float*>(p);
        p += align_up(stream_partial_bytes(static_cast<int>(T), static_cast<int>(H), static_cast<int>(E),
                                           static_cast<int>(K), static_cast<int>(I), stream_wide(T, H, E, K, I),
                                           splits.gateup), 256);
        ws.slot_row = reinterpret_cast<int32_t*>(p);
    } else if (schedule == 1) {
        ws.pscratch = reinterpret_cast<int32_t*>(p);
        p += align_up(permute_scratch_bytes(static_cast<int>(S), static_cast<int>(E)), 256);
        if (splits.tiled && tiled_partial_bytes(static_cast<int>(T), static_cast<int>(H), static_cast<int>(E),
                                               static_cast<int>(K), static_cast<int>(I)) > 0)
            ws.partial = reinterpret_cast<float*>(p);
    }
    return ws;
}

FfnGrid ffn_grid(int T, int H, int E, int K, int I) {
    FfnGrid g;
    g.schedule = ffn_schedule(T, H, E, K, I);
    if (g.schedule == 1) {
        g.block_threads = tiled_block_threads();
        g.gateup_blocks = tiled_gateup_grid(T, E, K, I);
        g.down_blocks = tiled_down_grid(T, E, K, H);
        g.rows_per_tile = tiled_rows_per_tile();
    } else {
        g.block_threads = stream_block_threads();
        g.gateup_blocks = stream_gateup_grid(T, H, E, K, I, stream_wide(T, H, E, K, I));
        g.down_blocks = stream_down_grid(T, H, E, K, I, stream_wide(T, H, E, K, I));
        g.rows_per_tile = stream_rows_per_pass();
    }
    return g;
}

hipError_t launch_ffn(const uint16_t* x, const int32_t* expert_ids, const uint16_t* expert_weights,
                      uint16_t* expert_out, FfnWorkspace ws, int T, int H, int E, int K, int I, hipStream_t stream,
                      FfnSplits splits) {
    switch (ffn_schedule(T, H, E, K, I, splits)) {
        case 1: {
            hipError_t err = prepare_permute(T * K, E);
            if (err == hipSuccess) err = prepare_ffn_tiled();
            if (err == hipSuccess) err = launch_permute(expert_ids, T * K, E, H, ws, expert_out, stream);
            if (err != hipSuccess) return err;
            return launch_ffn_tiled(x, expert_weights, expert_out, ws, T, H, E, K, I, stream, splits.tiled);
        }
        case 0: {
            const hipError_t err = prepare_ffn_stream(H, I);
            if (err != hipSuccess) return err;
            return launch_ffn_stream(x, expert_ids, expert_weights, expert_out, ws, T, H, E, K, I, stream, nullptr,
                                     nullptr, splits.gateup);
        }
        default: return hipErrorInvalidValue;
    }
}

hipError_t launch_ffn_combine(const uint16_t* x, const int32_t* expert_ids, const uint16_t* weights,
                              const uint16_t* expert_weights, uint16_t* expert_out, uint16_t* y, FfnWorkspace ws,
                              int T, int H, int E, int K, int I, hipStream_t stream) {
    if (ffn_schedule(T, H, E, K, I) == 0) {
        const hipError_t err = prepare_ffn_stream(H, I);
        if (err != hipSuccess) return err;
        return launch_ffn_stream(x, expert_ids, expert_weights, expert_out, ws, T, H, E, K, I, stream, weights, y);
    }
    const hipError_t err = launch_ffn(x, expert_ids, expert_weights, expert_out, ws, T, H, E, K, I, stream);
    if (err != hipSuccess) return err;
    return launch_combine(expert_out, weights, y, T, H, K, stream);
}

size_t layer_workspace_bytes(int64_t T, int64_t H, int64_t E, int64_t K, int64_t I) {
    size_t bytes = ffn_workspace_bytes(T, H, E, K, I);
    // counts for the routing blocks of any routing kernel: at most one block per 16 tokens
    if (ffn_schedule(T, H, E, K, I) == 1)
        bytes += align_up(sizeof(int32_t) * static_cast<size_t>((T + 15) / 16) * counts_stride(static_cast<int>(E)), 256);
    else  // the split routing's quarter sums (small batches, E > 64)
        bytes += align_up(routing_split_workspace_bytes(static_cast<int>(T), static_cast<int>(E)), 256);
    return bytes;
}

hipError_t launch_layer(const uint16_t* x, const uint16_t* w_gate, const uint16_t* expert_weights, int32_t* ids,
                        uint16_t* weights, uint16_t* expert_out, uint16_t* y, void* workspace, int T, int H, int E,
                        int K, int I, hipStream_t stream) {
    const FfnWorkspace ws = ffn_workspace_carve(workspace, T, H, E, K, I);
    switch (ffn_schedule(T, H, E, K, I)) {
        case 1: {
            hipError_t err = prepare_ffn_tiled();
            if (err != hipSuccess) return err;
            // rank [T*K] in the permute's scratch; the routing blocks' counts after the FFN workspace
            int32_t* rank = ws.pscratch;
            int32_t* counts = reinterpret_cast<int32_t*>(static_cast<char*>(workspace) + ffn_workspace_bytes(T, H, E, K, I));
            err = launch_routing_topk(x, w_gate, ids, weights, T, H, E, K, stream, counts, rank);
            if (err != hipSuccess) return err;
            const bool lw = routing_lds_weights(w_gate, H, E);  // the same choice the routing launch makes
            const int nblocks = routing_blocks(T, H, E, lw);
            err = launch_permute_scatter(ids, T * K, E, H, counts, rank, nblocks, routing_tokens_per_block(T, H, E, lw) * K,
                                         permute_scatter_chunks_per_block(nblocks), ws, expert_out, stream);
            if (err != hipSuccess) return err;
            err = launch_ffn_tiled(x, expert_weights, expert_out, ws, T, H, E, K, I, stream, /*allow_split=*/true);
            if (err != hipSuccess) return err;
            return launch_combine(expert_out, weights, y, T, H, K, stream);
        }
        case 0: {
            hipError_t err = prepare_ffn_stream(H, I);  // the FFN kernels' attributes before the first launch
            if (err != hipSuccess) return err;
            if (routing_split_applies(T, H, E, routing_lds_weights(w_gate, H, E))) {
                float* part = reinterpret_cast<float*>(static_cast<char*>(workspace) + ffn_workspace_bytes(T, H, E, K, I));
                err = launch_routing_split(x, w_gate, ids, weights, T, H, E, K, part, stream);
            } else {
                err = launch_routing_topk(x, w_gate, ids, weights, T, H, E, K, stream);
            }
            if (err != hipSuccess) return err;
            return launch_ffn_combine(x, ids, weights, expert_weights, expert_out, y, ws, T, H, E, K, I, stream);
        }
        default: return hipErrorInvalidValue;
    }
}

}  // namespace moe
