// moe_ops.cpp -- host side of libmoe_mi355x.so: the C ABI declared in include/moe_ops.h.
//
// Replaces op_host/moe_ops.cpp of the reference: operator argument checks (the TilingFuncs' GRAPH_FAILED
// paths), InferShape / InferDataType, launch planning (TilingFunc) and the launches themselves. Nothing here
// allocates device memory; every failure is reported before a kernel is queued.

#include <hip/hip_runtime.h>

#include <cstdarg>
#include <cstdio>
#include <cstring>

#include "moe_launch.h"
#include "moe_ops.h"
#include "moe_synth.h"

namespace {

thread_local char g_last_error[512] = "";

moe_status fail(moe_status st, const char* fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    std::vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
    va_end(ap);
    return st;
}

moe_status ok() {
    g_last_error[0] = '\0';
    return MOE_OK;
}

moe_status hip_fail(hipError_t err, const char* what) {
    return fail(MOE_ERR_HIP, "%s: %s", what, hipGetErrorString(err));
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

constexpr int64_t kMaxExperts = 256;
constexpr int64_t kInt32Max = 2147483647;
// hiddenSize and intermediateSize bound: far above any model's, and small enough that the products of sizes the
// checks below form stay within 64 bits
constexpr int64_t kMaxDim = int64_t{1} << 20;

// a * b > limit for a, b >= 0, without forming a product that could overflow
bool product_exceeds(int64_t a, int64_t b, int64_t limit) { return b != 0 && a > limit / b; }

// Scalar checks shared by the planners and launches.
moe_status check_routing_sizes(int64_t T, int64_t H, int64_t E, int64_t K) {
    if (T < 0 || H <= 0 || E <= 0) return fail(MOE_ERR_ARG, "sizes must be T >= 0, H > 0, E > 0 (T=%lld H=%lld E=%lld)",
                                               (long long)T, (long long)H, (long long)E);
    if (K < 1 || K > E) return fail(MOE_ERR_ARG, "topK=%lld must be in [1, numExperts=%lld]", (long long)K, (long long)E);
    if (H % 32 != 0) return fail(MOE_ERR_UNSUPPORTED, "hiddenSize=%lld must be a multiple of 32", (long long)H);
    if (E > kMaxExperts) return fail(MOE_ERR_UNSUPPORTED, "numExperts=%lld exceeds %lld", (long long)E, (long long)kMaxExperts);
    if (H > kMaxDim) return fail(MOE_ERR_UNSUPPORTED, "hiddenSize=%lld exceeds %lld", (long long)H, (long long)kMaxDim);
    if (product_exceeds(T, H, kInt32Max * 8LL) || product_exceeds(T, K, kInt32Max))
        return fail(MOE_ERR_UNSUPPORTED, "T=%lld too large", (long long)T);
    return ok();
}

moe_status check_ffn_sizes(int64_t T, int64_t H, int64_t E, int64_t K, int64_t I) {
    moe_status st = check_routing_sizes(T, H, E, K);
    if (st != MOE_OK) return st;
    if (I <= 0) return fail(MOE_ERR_ARG, "intermediateSize=%lld must be > 0", (long long)I);
    if (I % 32 != 0) return fail(MOE_ERR_UNSUPPORTED, "intermediateSize=%lld must be a multiple of 32", (long long)I);
    if (I > kMaxDim)
        return fail(MOE_ERR_UNSUPPORTED, "intermediateSize=%lld exceeds %lld", (long long)I, (long long)kMaxDim);
    if (moe::ffn_schedule(T, H, E, K, I) < 0) {
        if (moe::tiled_shape_supported(H, E, I) && !moe::tiled_size_supported(T, H, K, I))
            return fail(MOE_ERR_UNSUPPORTED,
                        "T=%lld H=%lld K=%lld I=%lld exceeds the tiled expert GEMMs' 32-bit buffer offsets (x, one "
                        "expert's weights and the sorted slots must each stay below 2 GiB)",
                        (long long)T, (long long)H, (long long)K, (long long)I);
        return fail(MOE_ERR_UNSUPPORTED, "hiddenSize=%lld / intermediateSize=%lld: no expert GEMM schedule fits",
                    (long long)H, (long long)I);
    }
    if (product_exceeds(T * K, I, kInt32Max * 64LL)) return fail(MOE_ERR_UNSUPPORTED, "T*K*I too large");  // T*K <= 2^31
    return ok();
}

moe_status check_combine_sizes(int64_t T, int64_t H, int64_t K) {
    if (T < 0 || H <= 0 || K < 1)
        return fail(MOE_ERR_ARG, "sizes must be T >= 0, H > 0, K >= 1 (T=%lld H=%lld K=%lld)", (long long)T,
                    (long long)H, (long long)K);
    if (H % 8 != 0) return fail(MOE_ERR_UNSUPPORTED, "hiddenSize=%lld must be a multiple of 8", (long long)H);
    if (H > kMaxDim) return fail(MOE_ERR_UNSUPPORTED, "hiddenSize=%lld exceeds %lld", (long long)H, (long long)kMaxDim);
    if (product_exceeds(T, K, kInt32Max)) return fail(MOE_ERR_UNSUPPORTED, "T*K too large");
    return ok();
}

hipStream_t as_stream(void* s) { return static_cast<hipStream_t>(s); }

}  // namespace

extern "C" {

const char* moe_status_string(moe_status status) {
    switch (status) {
        case MOE_OK: return "MOE_OK";
        case MOE_ERR_NULL: return "MOE_ERR_NULL";
        case MOE_ERR_RANK: return "MOE_ERR_RANK";
        case MOE_ERR_SHAPE: return "MOE_ERR_SHAPE";
        case MOE_ERR_ARG: return "MOE_ERR_ARG";
        case MOE_ERR_WORKSPACE: return "MOE_ERR_WORKSPACE";
        case MOE_ERR_UNSUPPORTED: return "MOE_ERR_UNSUPPORTED";
        case MOE_ERR_HIP: return "MOE_ERR_HIP";
    }
    return "MOE_ERR_UNKNOWN";
}

const char* moe_last_error(void) { return g_last_error; }

const char* moe_version(void) { return "moe_mi355x 0.1.0 (gfx950)"; }

// ------------------------------------------------------------------------------------------------
// MoeRoutingTopK
// ------------------------------------------------------------------------------------------------

moe_status moe_routing_topk_infer_shape(const int64_t* x_dims, int32_t x_rank, const int64_t* w_gate_dims,
                                        int32_t w_gate_rank, int64_t top_k, int64_t expert_ids_dims[2],
                                        int64_t weights_dims[2]) {
    if (!x_dims || !w_gate_dims || !expert_ids_dims || !weights_dims)
        return fail(MOE_ERR_NULL, "MoeRoutingTopK: input shape is null");
    if (x_rank != 2 || w_gate_rank != 2)
        return fail(MOE_ERR_RANK, "MoeRoutingTopK: x rank=%d (expected 2), w_gate rank=%d (expected 2)", x_rank,
                    w_gate_rank);
    if (x_dims[1] != w_gate_dims[0])
        return fail(MOE_ERR_SHAPE, "MoeRoutingTopK: hiddenSize mismatch x[%lld] vs w_gate[%lld]",
                    (long long)x_dims[1], (long long)w_gate_dims[0]);
    const int64_t k = top_k > 0 ? top_k : 2;
    if (k > w_gate_dims[1])
        return fail(MOE_ERR_ARG, "MoeRoutingTopK: topK=%lld exceeds numExperts=%lld", (long long)k,
                    (long long)w_gate_dims[1]);
    expert_ids_dims[0] = weights_dims[0] = x_dims[0];
    expert_ids_dims[1] = weights_dims[1] = k;
    return ok();
}

moe_status moe_routing_topk_infer_dtype(moe_dtype* expert_ids_dtype, moe_dtype* weights_dtype) {
    if (!expert_ids_dtype || !weights_dtype) return fail(MOE_ERR_NULL, "MoeRoutingTopK: null dtype output");
    *expert_ids_dtype = MOE_DT_INT32;
    *weights_dtype = MOE_DT_FLOAT16;
    return ok();
}

moe_status moe_routing_topk_plan(int64_t T, int64_t H, int64_t E, int64_t K, moe_routing_plan* plan) {
    if (!plan) return fail(MOE_ERR_NULL, "MoeRoutingTopK: null plan");
    moe_status st = check_routing_sizes(T, H, E, K);
    if (st != MOE_OK) return st;
    plan->num_tokens = T;
    plan->hidden_size = H;
    plan->num_experts = E;
    plan->top_k = K;
    // the plan assumes a 16-byte aligned w_gate (hipMalloc memory is); the launch checks the pointer itself
    const bool lw = E % 8 == 0;
    plan->tokens_per_block =
        moe::routing_tokens_per_block(static_cast<int>(T), static_cast<int>(H), static_cast<int>(E), lw);
    plan->grid = static_cast<int32_t>((T + plan->tokens_per_block - 1) / plan->tokens_per_block);
    plan->block = moe::routing_block_threads(static_cast<int>(T), static_cast<int>(H), static_cast<int>(E), lw);
    plan->lds_bytes = moe::routing_lds_bytes(static_cast<int>(T), static_cast<int>(H), static_cast<int>(E), lw);
    plan->workspace_bytes = 0;
    return ok();
}

moe_status moe_routing_topk(const uint16_t* x, const uint16_t* w_gate, int32_t* expert_ids, uint16_t* weights,
                            int64_t T, int64_t H, int64_t E, int64_t K, void* stream) {
    moe_status st = check_routing_sizes(T, H, E, K);
    if (st != MOE_OK) return st;
    if (T == 0) return ok();
    if (!x || !w_gate || !expert_ids || !weights) return fail(MOE_ERR_NULL, "MoeRoutingTopK: null tensor pointer");
    if (!aligned16(x)) return fail(MOE_ERR_UNSUPPORTED, "MoeRoutingTopK: x must be 16-byte aligned");
    hipError_t err = moe::launch_routing_topk(x, w_gate, expert_ids, weights, static_cast<int>(T),
                                              static_cast<int>(H), static_cast<int>(E), static_cast<int>(K),
                                              as_stream(stream));
    if (err != hipSuccess) return hip_fail(err, "MoeRoutingTopK launch");
    return ok();
}

// ------------------------------------------------------------------------------------------------
// MoeExpertFFN
// ------------------------------------------------------------------------------------------------

moe_status moe_expert_ffn_infer_shape(const int64_t* x_dims, int32_t x_rank, const int64_t* expert_ids_dims,
                                      int32_t expert_ids_rank, const int64_t* expert_weights_dims,
                                      int32_t expert_weights_rank, int64_t intermediate_size_attr,
                                      int64_t expert_out_dims[3], int64_t* intermediate_size) {
    if (!x_dims || !expert_ids_dims || !expert_weights_dims || !expert_out_dims)
        return fail(MOE_ERR_NULL, "MoeExpertFFN: input shape is null");
    if (x_rank != 2) return fail(MOE_ERR_RANK, "MoeExpertFFN: x must be 2D, got rank %d", x_rank);
    if (expert_ids_rank != 2)
        return fail(MOE_ERR_RANK, "MoeExpertFFN: expert_ids must be 2D, got rank %d", expert_ids_rank);
    if (expert_weights_rank != 3)
        return fail(MOE_ERR_RANK, "MoeExpertFFN: expert_weights must be 3D, got rank %d", expert_weights_rank);
    if (expert_ids_dims[0] != x_dims[0])
        return fail(MOE_ERR_SHAPE, "MoeExpertFFN: expert_ids[%lld] vs x[%lld] token count mismatch",
                    (long long)expert_ids_dims[0], (long long)x_dims[0]);
    if (expert_weights_dims[2] != x_dims[1])
        return fail(MOE_ERR_SHAPE, "MoeExpertFFN: hiddenSize mismatch x[%lld] vs expert_weights[%lld]",
                    (long long)x_dims[1], (long long)expert_weights_dims[2]);
    if (expert_weights_dims[1] % 3 != 0)
        return fail(MOE_ERR_SHAPE, "MoeExpertFFN: expert_weights dim 1 (%lld) is not 3*intermediateSize",
                    (long long)expert_weights_dims[1]);
    int64_t inter = expert_weights_dims[1] / 3;
    if (intermediate_size_attr > 0 && intermediate_size_attr != inter)
        return fail(MOE_ERR_SHAPE, "MoeExpertFFN: intermediateSize attr %lld disagrees with expert_weights (%lld)",
                    (long long)intermediate_size_attr, (long long)inter);
    expert_out_dims[0] = x_dims[0];
    expert_out_dims[1] = expert_ids_dims[1];
    expert_out_dims[2] = x_dims[1];
    if (intermediate_size) *intermediate_size = inter;
    return ok();
}

moe_status moe_expert_ffn_infer_dtype(moe_dtype* expert_out_dtype) {
    if (!expert_out_dtype) return fail(MOE_ERR_NULL, "MoeExpertFFN: null dtype output");
    *expert_out_dtype = MOE_DT_FLOAT16;
    return ok();
}

size_t moe_expert_ffn_workspace_bytes(int64_t T, int64_t H, int64_t E, int64_t K, int64_t I) {
    if (check_ffn_sizes(T, H, E, K, I) != MOE_OK) return 0;
    return moe::ffn_workspace_bytes(T, H, E, K, I);
}

moe_status moe_expert_ffn_plan(int64_t T, int64_t H, int64_t E, int64_t K, int64_t I, moe_ffn_plan* plan) {
    if (!plan) return fail(MOE_ERR_NULL, "MoeExpertFFN: null plan");
    moe_status st = check_ffn_sizes(T, H, E, K, I);
    if (st != MOE_OK) return st;
    const moe::FfnGrid g = moe::ffn_grid(static_cast<int>(T), static_cast<int>(H), static_cast<int>(E),
                                         static_cast<int>(K), static_cast<int>(I));
    plan->num_tokens = T;
    plan->hidden_size = H;
    plan->num_experts = E;
    plan->top_k = K;
    plan->intermediate_size = I;
    plan->schedule = g.schedule;
    plan->permute_grid = g.schedule == 1 ? moe::permute_chunks(static_cast<int>(T * K)) : 0;
    plan->gateup_grid = g.gateup_blocks;
    plan->down_grid = g.down_blocks;
    plan->block = g.block_threads;
    plan->rows_per_tile = g.rows_per_tile;
    plan->workspace_bytes = moe::ffn_workspace_bytes(T, H, E, K, I);
    return ok();
}

moe_status moe_expert_ffn(const uint16_t* x, const int32_t* expert_ids, const uint16_t* weights,
                          const uint16_t* expert_weights, uint16_t* expert_out, void* workspace,
                          size_t workspace_bytes, int64_t T, int64_t H, int64_t E, int64_t K, int64_t I,
                          void* stream) {
    (void)weights;  // part of the operator signature; the FFN math does not use the routing weights
    moe_status st = check_ffn_sizes(T, H, E, K, I);
    if (st != MOE_OK) return st;
    if (T == 0) return ok();
    if (!x || !expert_ids || !expert_weights || !expert_out)
        return fail(MOE_ERR_NULL, "MoeExpertFFN: null tensor pointer");
    const size_t need = moe::ffn_workspace_bytes(T, H, E, K, I);
    if (!workspace || workspace_bytes < need)
        return fail(MOE_ERR_WORKSPACE, "MoeExpertFFN: workspace %zu bytes at %p, need %zu", workspace_bytes,
                    workspace, need);
    if (!aligned16(x) || !aligned16(expert_weights) || !aligned16(expert_out) || !aligned16(workspace))
        return fail(MOE_ERR_UNSUPPORTED, "MoeExpertFFN: x, expert_weights, expert_out, workspace must be 16-byte aligned");
    const hipStream_t s = as_stream(stream);
    const moe::FfnWorkspace ws = moe::ffn_workspace_carve(workspace, T, H, E, K, I);
    const hipError_t err = moe::launch_ffn(x, expert_ids, expert_weights, expert_out, ws, static_cast<int>(T),
                                           static_cast<int>(H), static_cast<int>(E), static_cast<int>(K),
                                           static_cast<int>(I), s);
    if (err != hipSuccess) return hip_fail(err, "MoeExpertFFN GEMM launch");
    return ok();
}

// MoeExpertFFN with the library's fixed per-GPU scratch as its workspace (no allocation anywhere)
moe_status moe_expert_ffn_no_alloc(const uint16_t* x, const int32_t* expert_ids, const uint16_t* weights,
                                   const uint16_t* expert_weights, uint16_t* expert_out, int64_t T, int64_t H,
                                   int64_t E, int64_t K, int64_t I, void* stream) {
    (void)weights;  // part of the operator signature; the FFN math does not use the routing weights
    moe_status st = check_ffn_sizes(T, H, E, K, I);
    if (st != MOE_OK) return st;
    if (T == 0) return ok();
    if (!x || !expert_ids || !expert_weights || !expert_out)
        return fail(MOE_ERR_NULL, "MoeExpertFFN (no alloc): null tensor pointer");
    if (!aligned16(x) || !aligned16(expert_weights) || !aligned16(expert_out))
        return fail(MOE_ERR_UNSUPPORTED, "MoeExpertFFN (no alloc): x, expert_weights, expert_out must be 16-byte aligned");
    // the tiled schedule runs its down projection unsplit here (its split partial tiles alone take up to 64 MiB);
    // the streaming gate/up kernel splits a long H only if its partial sums fit, else the call runs that H unsplit
    moe::FfnSplits splits;
    splits.tiled = false;
    size_t need = moe::ffn_workspace_bytes(T, H, E, K, I, splits);
    if (need > moe::noalloc_scratch_bytes()) {
        moe::FfnSplits compact = splits;
        compact.gateup = false;
        if (moe::ffn_schedule(T, H, E, K, I, compact) >= 0 &&
            moe::ffn_workspace_bytes(T, H, E, K, I, compact) <= moe::noalloc_scratch_bytes()) {
            splits = compact;
            need = moe::ffn_workspace_bytes(T, H, E, K, I, splits);
        }
    }
    if (need > moe::noalloc_scratch_bytes())
        return fail(MOE_ERR_UNSUPPORTED,
                    "MoeExpertFFN (no alloc): T=%lld H=%lld E=%lld K=%lld I=%lld needs %zu bytes of workspace, the "
                    "fixed scratch holds %zu; use moe_expert_ffn with a caller workspace",
                    (long long)T, (long long)H, (long long)E, (long long)K, (long long)I, need,
                    moe::noalloc_scratch_bytes());
    void* scratch = nullptr;
    hipError_t err = moe::noalloc_scratch(&scratch);
    if (err != hipSuccess) return hip_fail(err, "MoeExpertFFN (no alloc): scratch address");
    const moe::FfnWorkspace ws = moe::ffn_workspace_carve(scratch, T, H, E, K, I, splits);
    err = moe::launch_ffn(x, expert_ids, expert_weights, expert_out, ws, static_cast<int>(T), static_cast<int>(H),
                          static_cast<int>(E), static_cast<int>(K), static_cast<int>(I), as_stream(stream), splits);
    if (err != hipSuccess) return hip_fail(err, "MoeExpertFFN (no alloc) GEMM launch");
    return ok();
}

// MoeExpertFFN + MoeCombine in one call (optional fast path; both operators stay the contract)
moe_status moe_expert_ffn_combine(const uint16_t* x, const int32_t* expert_ids, const uint16_t* weights,
                                  const uint16_t* expert_weights, uint16_t* expert_out, uint16_t* y,
                                  void* workspace, size_t workspace_bytes, int64_t T, int64_t H, int64_t E, int64_t K,
                                  int64_t I, void* stream) {
    moe_status st = check_ffn_sizes(T, H, E, K, I);
    if (st != MOE_OK) return st;
    st = check_combine_sizes(T, H, K);
    if (st != MOE_OK) return st;
    if (T == 0) return ok();
    if (!x || !expert_ids || !weights || !expert_weights || !expert_out || !y)
        return fail(MOE_ERR_NULL, "MoeExpertFFN+MoeCombine: null tensor pointer");
    const size_t need = moe::ffn_workspace_bytes(T, H, E, K, I);
    if (!workspace || workspace_bytes < need)
        return fail(MOE_ERR_WORKSPACE, "MoeExpertFFN+MoeCombine: workspace %zu bytes at %p, need %zu", workspace_bytes,
                    workspace, need);
    if (!aligned16(x) || !aligned16(expert_weights) || !aligned16(expert_out) || !aligned16(workspace) ||
        !aligned16(y))
        return fail(MOE_ERR_UNSUPPORTED,
                    "MoeExpertFFN+MoeCombine: x, expert_weights, expert_out, y, workspace must be 16-byte aligned");
    const hipStream_t s = as_stream(stream);
    const moe::FfnWorkspace ws = moe::ffn_workspace_carve(workspace, T, H, E, K, I);
    const hipError_t err = moe::launch_ffn_combine(x, expert_ids, weights, expert_weights, expert_out, y, ws,
                                                   static_cast<int>(T), static_cast<int>(H), static_cast<int>(E),
                                                   static_cast<int>(K), static_cast<int>(I), s);
    if (err != hipSuccess) return hip_fail(err, "MoeExpertFFN+MoeCombine launch");
    return ok();
}

// The whole layer in one call (optional fast path; the three operators stay the contract)
size_t moe_layer_workspace_bytes(int64_t T, int64_t H, int64_t E, int64_t K, int64_t I) {
    if (check_ffn_sizes(T, H, E, K, I) != MOE_OK) return 0;
    return moe::layer_workspace_bytes(T, H, E, K, I);
}

moe_status moe_layer(const uint16_t* x, const uint16_t* w_gate, const uint16_t* expert_weights, int32_t* expert_ids,
                     uint16_t* weights, uint16_t* expert_out, uint16_t* y, void* workspace, size_t workspace_bytes,
                     int64_t T, int64_t H, int64_t E, int64_t K, int64_t I, void* stream) {
    moe_status st = check_ffn_sizes(T, H, E, K, I);  // includes the routing checks
    if (st != MOE_OK) return st;
    st = check_combine_sizes(T, H, K);
    if (st != MOE_OK) return st;
    if (T == 0) return ok();
    if (!x || !w_gate || !expert_weights || !expert_ids || !weights || !expert_out || !y)
        return fail(MOE_ERR_NULL, "MoE layer: null tensor pointer");
    const size_t need = moe::layer_workspace_bytes(T, H, E, K, I);
    if (!workspace || workspace_bytes < need)
        return fail(MOE_ERR_WORKSPACE, "MoE layer: workspace %zu bytes at %p, need %zu", workspace_bytes, workspace,
                    need);
    if (!aligned16(x) || !aligned16(expert_weights) || !aligned16(expert_out) || !aligned16(workspace) ||
        !aligned16(y))
        return fail(MOE_ERR_UNSUPPORTED, "MoE layer: x, expert_weights, expert_out, y, workspace must be 16-byte aligned");
    const hipError_t err = moe::launch_layer(x, w_gate, expert_weights, expert_ids, weights, expert_out, y, workspace,
                                             static_cast<int>(T), static_cast<int>(H), static_cast<int>(E),
                                             static_cast<int>(K), static_cast<int>(I), as_stream(stream));
    if (err != hipSuccess) return hip_fail(err, "MoE layer launch");
    return ok();
}

// ------------------------------------------------------------------------------------------------
// MoeCombine
// ------------------------------------------------------------------------------------------------

moe_status moe_combine_infer_shape(const int64_t* expert_out_dims, int32_t expert_out_rank,
                                   const int64_t* expert_ids_dims, int32_t expert_ids_rank, int64_t y_dims[2]) {
    if (!expert_out_dims || !y_dims) return fail(MOE_ERR_NULL, "MoeCombine: input shape is null");
    if (expert_out_rank != 3)
        return fail(MOE_ERR_RANK, "MoeCombine: expert_out must be 3D, got rank %d", expert_out_rank);
    if (expert_ids_dims) {
        if (expert_ids_rank != 2)
            return fail(MOE_ERR_RANK, "MoeCombine: expert_ids must be 2D, got rank %d", expert_ids_rank);
        if (expert_ids_dims[0] != expert_out_dims[0] || expert_ids_dims[1] != expert_out_dims[1])
            return fail(MOE_ERR_SHAPE, "MoeCombine: expert_ids [%lld, %lld] vs expert_out [%lld, %lld, *]",
                        (long long)expert_ids_dims[0], (long long)expert_ids_dims[1], (long long)expert_out_dims[0],
                        (long long)expert_out_dims[1]);
    }
    y_dims[0] = expert_out_dims[0];
    y_dims[1] = expert_out_dims[2];
    return ok();
}

moe_status moe_combine_infer_dtype(moe_dtype* y_dtype) {
    if (!y_dtype) return fail(MOE_ERR_NULL, "MoeCombine: null dtype output");
    *y_dtype = MOE_DT_FLOAT16;
    return ok();
}

moe_status moe_combine_plan_for(int64_t T, int64_t H, int64_t K, moe_combine_plan* plan) {
    if (!plan) return fail(MOE_ERR_NULL, "MoeCombine: null plan");
    moe_status st = check_combine_sizes(T, H, K);
    if (st != MOE_OK) return st;
    plan->num_tokens = T;
    plan->hidden_size = H;
    plan->top_k = K;
    plan->grid = moe::combine_grid(T, H);
    plan->block = moe::combine_block_threads();
    plan->elems_per_thread = moe::combine_elems_per_thread();
    plan->workspace_bytes = 0;
    return ok();
}

moe_status moe_combine(const uint16_t* expert_out, const int32_t* expert_ids, const uint16_t* weights, uint16_t* y,
                       int64_t T, int64_t H, int64_t K, void* stream) {
    (void)expert_ids;  // part of the operator signature; unused by the math (op_kernel/moe_combine.cpp:6)
    moe_status st = check_combine_sizes(T, H, K);
    if (st != MOE_OK) return st;
    if (T == 0) return ok();
    if (!expert_out || !weights || !y) return fail(MOE_ERR_NULL, "MoeCombine: null tensor pointer");
    if (!aligned16(expert_out) || !aligned16(y))
        return fail(MOE_ERR_UNSUPPORTED, "MoeCombine: expert_out and y must be 16-byte aligned");
    hipError_t err = moe::launch_combine(expert_out, weights, y, static_cast<int>(T), static_cast<int>(H),
                                         static_cast<int>(K), as_stream(stream));
    if (err != hipSuccess) return hip_fail(err, "MoeCombine launch");
    return ok();
}

// ------------------------------------------------------------------------------------------------
// Synthetic inputs / calibration (moe_synth.h)
// ------------------------------------------------------------------------------------------------

moe_status moe_synth_normal_f16(uint16_t* out, uint64_t n, uint64_t seed, uint64_t stream_id, double sigma_a,
                                double sigma_b, uint64_t period, uint64_t split, void* stream) {
    if (n == 0) return ok();
    if (!out) return fail(MOE_ERR_NULL, "moe_synth_normal_f16: null output");
    hipError_t err = moe::launch_synth_normal_f16(out, n, seed, stream_id, sigma_a, sigma_b, period, split,
                                                  as_stream(stream));
    if (err != hipSuccess) return hip_fail(err, "moe_synth_normal_f16 launch");
    return ok();
}

moe_status moe_copy_bytes(void* dst, const void* src, uint64_t bytes, void* stream) {
    if (bytes == 0) return ok();
    if (!dst || !src) return fail(MOE_ERR_NULL, "moe_copy_bytes: null pointer");
    if (bytes % 16 != 0 || !aligned16(dst) || !aligned16(src))
        return fail(MOE_ERR_ARG, "moe_copy_bytes: size and pointers must be multiples of 16");
    hipError_t err = moe::launch_copy_bytes(dst, src, bytes, as_stream(stream));
    if (err != hipSuccess) return hip_fail(err, "moe_copy_bytes launch");
    return ok();
}

moe_status moe_stream_read_bytes(const void* src, uint64_t bytes, void* stream) {
    if (bytes == 0) return ok();
    if (!src) return fail(MOE_ERR_NULL, "moe_stream_read_bytes: null pointer");
    if (bytes % 16384 != 0 || !aligned16(src))
        return fail(MOE_ERR_ARG, "moe_stream_read_bytes: size must be a multiple of 16384, pointer 16-byte aligned");
    hipError_t err = moe::launch_stream_read(src, bytes, as_stream(stream));
    if (err != hipSuccess) return hip_fail(err, "moe_stream_read_bytes launch");
    return ok();
}

}  // extern "C"
