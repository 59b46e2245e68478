// moe_launch.h -- internal interface between the C-ABI host layer (moe_ops.cpp) and the kernel files.
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

namespace moe {

constexpr int kRankTopK = 32;  // topK up to which the routing tail ranks its block's slots in one pass

// Per-kernel HIP-event timing (moe_trace.h). A TraceScope brackets exactly one kernel launch.
class TraceScope {
  public:
    TraceScope(const char* name, hipStream_t stream);
    ~TraceScope();
    TraceScope(const TraceScope&) = delete;
    TraceScope& operator=(const TraceScope&) = delete;

  private:
    const char* name_;
    hipStream_t stream_;
    hipEvent_t start_ = nullptr;
};

// ---- per-device launch preparation (moe_runtime.cpp) ----
// Raises kernel `fn`'s dynamic-LDS limit to `lds_max` bytes on the current device (once per device and kernel;
// needed above 64 KB). Returns the HIP error of that call, hipSuccess when it was already done.
hipError_t ensure_lds_limit(const void* fn, int lds_max);
// Workgroups of `fn` (`threads` threads, `lds` bytes of dynamic LDS) the current device holds at once, cached per
// device, kernel and LDS size; 0 when the device cannot be queried.
int resident_workgroups(const void* fn, int threads, size_t lds);

// ---- routing (moe_routing.hip) ----
int routing_expert_blocks(int E);
// lw: w_gate's rows can reach LDS 16 bytes at a time (E % 8 == 0, 16-byte aligned w_gate): routing_lds_weights
bool routing_lds_weights(const void* w_gate, int H, int E);
// moe_layer's routing of a batch of at most 16 tokens with E > 64: the quarters kernel's work over 4 * E / 32
// workgroups, the fp32 quarter sums in `part` (routing_split_workspace_bytes), the same ids and weights
bool routing_split_applies(int T, int H, int E, bool lw);
size_t routing_split_workspace_bytes(int T, int E);
hipError_t launch_routing_split(const uint16_t* x, const uint16_t* w_gate, int32_t* ids, uint16_t* w, int T, int H,
                                int E, int K, float* part, hipStream_t stream);
int routing_tokens_per_block(int T, int H, int E, bool lw);
int routing_block_threads(int T, int H, int E, bool lw);
int routing_lds_bytes(int T, int H, int E, bool lw);
int routing_blocks(int T, int H, int E, bool lw);  // workgroups of a launch, routing_tokens_per_block tokens each
// counts/rank non-null: the kernel's tail also ranks each block's slots by expert (rank[T*K]) and writes the
// block's per-expert counts (counts[routing_blocks][counts_stride(E)], 16-byte aligned), the permute's first half
hipError_t launch_routing_topk(const uint16_t* x, const uint16_t* w_gate, int32_t* ids, uint16_t* w, int T, int H,
                               int E, int K, hipStream_t stream, int32_t* counts = nullptr,
                               int32_t* rank = nullptr);

// ---- expert FFN (moe_permute.hip, moe_ffn.hip) ----
struct FfnWorkspace {
    int32_t* offsets;      // [E + 1] first sorted row of each expert; offsets[E] = number of valid slots
    int32_t* sorted_slot;  // [T*K]   slot index t*K + k of each sorted row, experts ascending, slots ascending
    uint16_t* hidden;      // [T*K, I] fp16 SwiGLU intermediate, rows in sorted order
    float* partial;        // fp32 split-K partial sums: [nsplit, T*K, H] of the streaming down projection, or the
                           // tiled schedule's partial tiles of its split leftover round
    int32_t* slot_row;     // [T*K]   sorted row of each slot with a valid id (weight-streaming schedule only)
    int32_t* pscratch;     // the permute's per-slot ranks and per-chunk counts (tiled schedule only)
};
// The split-K variants a call may use, both on by default: tiled = the tiled schedule's split leftover round of
// its down projection (up to 64 MiB of fp32 partial tiles), gateup = the 32-row streaming gate/up kernel's split
// of an H too long for LDS (splits x T*K x 2I fp32 partial sums). Off, the down projection runs unsplit and a
// long H runs 16-row streaming passes or the tiled schedule, with a smaller workspace.
struct FfnSplits {
    bool tiled = true;
    bool gateup = true;
};
size_t ffn_workspace_bytes(int64_t T, int64_t H, int64_t E, int64_t K, int64_t I, FfnSplits splits = {});
FfnWorkspace ffn_workspace_carve(void* base, int64_t T, int64_t H, int64_t E, int64_t K, int64_t I,
                                 FfnSplits splits = {});

int permute_block_threads();
int permute_chunks(int S);
size_t permute_scratch_bytes(int S, int E);
hipError_t prepare_permute(int S, int E);  // kernel attributes, before the first launch of a call
// the scatter alone, over chunk counts and ranks some other kernel wrote (counts rows of counts_stride(E) ints,
// 16-byte aligned; chunk c holds the slots [c chunk_slots, (c + 1) chunk_slots)), cpw chunks per workgroup
int permute_scatter_chunks_per_block(int nchunks);
hipError_t launch_permute_scatter(const int32_t* ids, int S, int E, int H, const int32_t* counts,
                                  const int32_t* rank, int nchunks, int chunk_slots, int cpw, FfnWorkspace ws,
                                  uint16_t* expert_out, hipStream_t stream);
hipError_t launch_permute(const int32_t* ids, int S, int E, int H, FfnWorkspace ws, uint16_t* expert_out,
                          hipStream_t stream);

struct FfnGrid {
    int gateup_blocks;
    int down_blocks;
    int block_threads;
    int rows_per_tile;
    int schedule;
};
FfnGrid ffn_grid(int T, int H, int E, int K, int I);
// weight-streaming schedule (moe_ffn_stream.hip)
int stream_block_threads();
int stream_rows_per_pass();
bool stream_supported(int H, int I, bool gateup_split = true);
// the wide weight-streaming kernels (up to 128 rows per pass): whether the shape allows them, and whether a call
// of this size runs them
bool stream_wide_supported(int H, int I);
bool stream_wide(int64_t T, int64_t H, int64_t E, int64_t K, int64_t I);
hipError_t prepare_ffn_stream(int H, int I);  // kernel attributes, before the first launch of a call
size_t stream_partial_bytes(int T, int H, int E, int K, int I, bool wide, bool gateup_split);
int stream_gateup_grid(int T, int H, int E, int K, int I, bool wide, bool gateup_split = true);
int stream_down_grid(int T, int H, int E, int K, int I, bool wide);
// with y non-null (and weights) the combine is produced too: by the split reduce when the down projection is
// split over K, else by the combine kernel after the FFN
hipError_t launch_ffn_stream(const uint16_t* x, const int32_t* expert_ids, const uint16_t* expert_weights,
                             uint16_t* expert_out, const FfnWorkspace& ws, int T, int H, int E, int K, int I,
                             hipStream_t stream, const uint16_t* weights = nullptr, uint16_t* y = nullptr,
                             bool gateup_split = true);
// LDS-tiled schedule (moe_ffn_tiled.hip)
bool tiled_shape_supported(int64_t H, int64_t E, int64_t I);           // H, I granularity and LDS
bool tiled_size_supported(int64_t T, int64_t H, int64_t K, int64_t I);  // 32-bit buffer offsets
bool tiled_supported(int64_t T, int64_t H, int64_t E, int64_t K, int64_t I);
hipError_t prepare_ffn_tiled();  // kernel attributes, before the first launch of a call
int tiled_block_threads();
// fp32 partial tiles of the down projection's split leftover round (workspace region after hidden)
size_t tiled_partial_bytes(int T, int H, int E, int K, int I);
int tiled_rows_per_tile();
int tiled_gateup_grid(int T, int E, int K, int I);
int tiled_down_grid(int T, int E, int K, int H);
// allow_split: the down projection may split its leftover tiles over k (needs ws.partial)
hipError_t launch_ffn_tiled(const uint16_t* x, const uint16_t* expert_weights, uint16_t* expert_out,
                            const FfnWorkspace& ws, int T, int H, int E, int K, int I, hipStream_t stream,
                            bool allow_split);
// schedule choice: 0 = weight streaming, 1 = LDS-tiled, -1 = no kernel supports the shape. A shape with many rows
// per expert that the tiled kernels support except for their 32-bit offsets is -1, not the streaming schedule
// (which would re-stream every expert's weights once per 32 rows).
int ffn_schedule(int64_t T, int64_t H, int64_t E, int64_t K, int64_t I, FfnSplits splits = {});
// the whole FFN: permute (tiled schedule; the streaming schedule finds rows itself) and the two GEMMs. Every
// kernel's attributes are set before the first launch, so a failure there leaves nothing launched.
hipError_t launch_ffn(const uint16_t* x, const int32_t* expert_ids, const uint16_t* expert_weights,
                      uint16_t* expert_out, FfnWorkspace ws, int T, int H, int E, int K, int I, hipStream_t stream,
                      FfnSplits splits = {});
// the FFN followed by the combine: expert_out as launch_ffn writes it, y as launch_combine would compute it
hipError_t launch_ffn_combine(const uint16_t* x, const int32_t* expert_ids, const uint16_t* weights,
                              const uint16_t* expert_weights, uint16_t* expert_out, uint16_t* y, FfnWorkspace ws,
                              int T, int H, int E, int K, int I, hipStream_t stream);

// ---- the whole layer: routing -> FFN -> combine in one call (moe_ffn.hip) ----
// workspace: the FFN's (ffn_workspace_bytes), then on the tiled schedule the routing blocks' expert counts
size_t layer_workspace_bytes(int64_t T, int64_t H, int64_t E, int64_t K, int64_t I);
// Tiled schedule: the routing kernel also ranks its blocks' slots (the permute's count), then one scatter launch,
// the two GEMMs and the combine. Streaming schedule: routing, then launch_ffn_combine. ids, weights, expert_out
// and y equal the three operators' bit for bit.
hipError_t launch_layer(const uint16_t* x, const uint16_t* w_gate, const uint16_t* expert_weights, int32_t* ids,
                        uint16_t* weights, uint16_t* expert_out, uint16_t* y, void* workspace, int T, int H, int E,
                        int K, int I, hipStream_t stream);

// ---- fixed scratch of the allocation-free FFN entry point (moe_noalloc.hip) ----
size_t noalloc_scratch_bytes();
// the current device's scratch array, looked up once per device (hipGetSymbolAddress with that device current)
hipError_t noalloc_scratch(void** ptr);

// ---- combine (moe_combine.hip) ----
int combine_block_threads();
int combine_elems_per_thread();
int combine_grid(int64_t T, int64_t H);
hipError_t launch_combine(const uint16_t* expert_out, const uint16_t* weights, uint16_t* y, int T, int H, int K,
                          hipStream_t stream);

// ---- synthetic inputs / calibration (moe_synth.hip) ----
hipError_t launch_synth_normal_f16(uint16_t* out, uint64_t n, uint64_t seed, uint64_t stream_id, double sigma_a,
                                   double sigma_b, uint64_t period, uint64_t split, hipStream_t stream);
hipError_t launch_copy_bytes(void* dst, const void* src, uint64_t bytes, hipStream_t stream);
hipError_t launch_stream_read(const void* src, uint64_t bytes, hipStream_t stream);

}  // namespace moe
