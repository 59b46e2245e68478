/*
 * moe_ops.h -- C ABI of the MI355X (gfx950) MoE operator library libmoe_mi355x.so.
 *
 * Drop-in for the three CANN operators of Lu-Yu-Zhen/Implementing-MoE-Architecture-Operators-on-CANN-Platform:
 *   MoeRoutingTopK -> MoeExpertFFN -> MoeCombine
 * Each CANN operator is one OpDef (prototype) + InferShape + InferDataType + TilingFunc in
 * op_host/moe_ops.cpp, and one kernel entry point in the op_kernel/ sources. Here each becomes a set of plain C
 * functions: *_infer_shape / *_infer_dtype (graph-time), *_plan (launch planning) and the launch itself.
 *
 * Conventions (kept from the reference, op_host/moe_ops.cpp and tests/test_moe.cpp:415-463):
 *   - All tensors are dense row-major ("ND"). fp16 tensors are passed as pointers to IEEE binary16 bit
 *     patterns (uint16_t storage); int32 tensors as int32_t.
 *   - The caller allocates and frees every device buffer, including the workspace; the library never
 *     allocates device memory. Launches are asynchronous and ordered on `stream` (a hipStream_t; NULL means
 *     the default stream); the caller synchronises.
 *   - Shape/argument errors are reported before anything is launched, as a moe_status (the reference's
 *     GRAPH_FAILED + OP_LOGE); moe_last_error() returns the message for the calling thread.
 *   - No host-side state is kept across calls (except the optional tracer in moe_trace.h): calls are
 *     re-entrant and may be issued from several threads on different streams.
 *
 * Expert weight layout (tests/moe_cpu_sim.cpp:174-179,254-260; tests/test_moe.cpp:200-201), per expert e,
 * with I = intermediate size and H = hidden size, in the single tensor expert_weights[E, 3*I, H]:
 *   W_gate[e][i][h] at e*3*I*H +         i*H + h   ([I, H] row-major)
 *   W_up  [e][i][h] at e*3*I*H +   I*H + i*H + h   ([I, H] row-major)
 *   W_down[e][h][i] at e*3*I*H + 2*I*H + h*I + i   ([H, I] row-major)
 * The reference's NPU kernel reads W_down as [I, H] (op_kernel/moe_expert_ffn.cpp:348-375); both of its CPU
 * references use [H, I], and this library follows the CPU references.
 *
 * Limits of the gfx950 kernels (MOE_ERR_UNSUPPORTED otherwise): H % 32 == 0, I % 32 == 0, H and I at most
 * 2^20, 1 <= K <= E <= 256, T*K < 2^31, and 16-byte aligned x, expert_weights, expert_out and y.
 * Calls with many rows per expert (the LDS-tiled schedule, moe_expert_ffn_plan .schedule == 1) also need
 * T*H*2 (x), 3*I*H*2 (one expert's weights) and T*K*4 (the sorted slots) below 2 GiB: the tiled kernels address
 * them with 32-bit buffer offsets. Such calls beyond those bounds are rejected with the reason rather than run
 * on the weight-streaming schedule, which would stream every expert's weights again for each 128 of its rows.
 * The tiled schedule also needs H > 64 and I > 64 (two k-stages of 64); an odd multiple of 32 ends with a
 * 32-column stage.
 */
#ifndef MOE_OPS_H
#define MOE_OPS_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef enum moe_status {
    MOE_OK = 0,
    MOE_ERR_NULL = 1,        /* required pointer is NULL (op_host/moe_ops.cpp:71-74,241-245,412-415)      */
    MOE_ERR_RANK = 2,        /* wrong tensor rank (op_host/moe_ops.cpp:80-85,251-258,421-428)             */
    MOE_ERR_SHAPE = 3,       /* inconsistent dims, e.g. hidden size mismatch (op_host/moe_ops.cpp:86-90)  */
    MOE_ERR_ARG = 4,         /* invalid scalar argument: sizes <= 0, topK outside [1, E]                  */
    MOE_ERR_WORKSPACE = 5,   /* workspace NULL or smaller than moe_expert_ffn_workspace_bytes()           */
    MOE_ERR_UNSUPPORTED = 6, /* valid request outside the gfx950 kernels' limits (see header comment)     */
    MOE_ERR_HIP = 7          /* a HIP runtime call or kernel launch failed                                */
} moe_status;

typedef enum moe_dtype {
    MOE_DT_FLOAT16 = 1, /* ge::DT_FLOAT16 */
    MOE_DT_INT32 = 3    /* ge::DT_INT32   */
} moe_dtype;

/* Human-readable name of a status code. */
const char* moe_status_string(moe_status status);
/* Message describing the last failure on the calling thread ("" if none). */
const char* moe_last_error(void);
/* Library version string. */
const char* moe_version(void);

/* ------------------------------------------------------------------------------------------------------
 * MoeRoutingTopK: x[T, H] fp16, w_gate[H, E] fp16 -> expert_ids[T, K] int32, weights[T, K] fp16.
 *   logits = x @ w_gate (fp32 accumulation), row softmax, top-K experts in descending probability order
 *   (exact ties: lowest expert index first), weights renormalised over the K chosen to sum to 1.
 *   Attr topK (default 2, op_host/moe_ops.cpp:565-567).
 * ---------------------------------------------------------------------------------------------------- */

/* InferShape (op_host/moe_ops.cpp:181-214): expert_ids and weights are [x_dims[0], top_k].
 * top_k <= 0 selects the attr default 2. Checks ranks and x_dims[1] == w_gate_dims[0]
 * (the TilingFunc check, op_host/moe_ops.cpp:80-90). */
moe_status moe_routing_topk_infer_shape(const int64_t* x_dims, int32_t x_rank, const int64_t* w_gate_dims,
                                        int32_t w_gate_rank, int64_t top_k, int64_t expert_ids_dims[2],
                                        int64_t weights_dims[2]);
/* InferDataType (op_host/moe_ops.cpp:219-226): INT32, FLOAT16. */
moe_status moe_routing_topk_infer_dtype(moe_dtype* expert_ids_dtype, moe_dtype* weights_dtype);

/* Launch plan (TilingFunc replacement, op_host/moe_ops.cpp:63-176; TilingData op_host/moe_tiling.h:27-43). */
typedef struct moe_routing_plan {
    int64_t num_tokens, hidden_size, num_experts, top_k;
    int32_t tokens_per_block; /* tokens handled by one workgroup                        */
    int32_t grid;             /* workgroups                                             */
    int32_t block;            /* threads per workgroup                                  */
    int32_t lds_bytes;        /* dynamic LDS per workgroup                              */
    size_t workspace_bytes;   /* always 0, as in the reference (op_host/moe_ops.cpp:164-167) */
} moe_routing_plan;
moe_status moe_routing_topk_plan(int64_t num_tokens, int64_t hidden_size, int64_t num_experts, int64_t top_k,
                                 moe_routing_plan* plan);

/* Kernel entry MoeRoutingTopK(x, wGate, expertIds, weights, tiling) (op_kernel/moe_routing.cpp:434-440). */
moe_status moe_routing_topk(const uint16_t* x, const uint16_t* w_gate, int32_t* expert_ids, uint16_t* weights,
                            int64_t num_tokens, int64_t hidden_size, int64_t num_experts, int64_t top_k,
                            void* stream);

/* ------------------------------------------------------------------------------------------------------
 * MoeExpertFFN: x[T, H] fp16, expert_ids[T, K] int32, weights[T, K] fp16 (not used by the math, kept for
 *   signature parity), expert_weights[E, 3*I, H] fp16 -> expert_out[T, K, H] fp16.
 *   expert_out[t, k, :] = W_down_e @ (silu(W_gate_e @ x_t) * (W_up_e @ x_t)), e = expert_ids[t, k],
 *   fp32 accumulation; the SwiGLU intermediate is kept in fp16 in the workspace.
 *   Ids outside [0, E) are not computed: their expert_out rows are written as zeros.
 *   Attr intermediateSize (default 8192, op_host/moe_ops.cpp:618-620).
 * ---------------------------------------------------------------------------------------------------- */

/* InferShape (op_host/moe_ops.cpp:364-388): expert_out is [x_dims[0], expert_ids_dims[1], x_dims[1]].
 * The intermediate size is expert_weights_dims[1] / 3, overridden by intermediate_size_attr when > 0, as the
 * TilingFunc does (op_host/moe_ops.cpp:264-278); unlike the reference an override that disagrees with
 * expert_weights_dims[1] is rejected (MOE_ERR_SHAPE) instead of reading past the weights.
 * *intermediate_size receives the resolved value. */
moe_status moe_expert_ffn_infer_shape(const int64_t* x_dims, int32_t x_rank, const int64_t* expert_ids_dims,
                                      int32_t expert_ids_rank, const int64_t* expert_weights_dims,
                                      int32_t expert_weights_rank, int64_t intermediate_size_attr,
                                      int64_t expert_out_dims[3], int64_t* intermediate_size);
/* InferDataType (op_host/moe_ops.cpp:393-398): FLOAT16. */
moe_status moe_expert_ffn_infer_dtype(moe_dtype* expert_out_dtype);

/* Workspace bytes for one call (TilingFunc workspace, op_host/moe_ops.cpp:340-349). Holds the expert-sorted
 * slot order, per-expert offsets and the fp16 SwiGLU intermediate [T*K, I]; on the weight-streaming schedule
 * also the split-K partial sums and the slot -> sorted-row map; on the LDS-tiled schedule also up to 64 MiB of
 * fp32 partial tiles for the tiles it splits over k (only when its down tiles fill at most 4 rounds of the
 * GPU). 0 for invalid sizes. */
size_t moe_expert_ffn_workspace_bytes(int64_t num_tokens, int64_t hidden_size, int64_t num_experts,
                                      int64_t top_k, int64_t intermediate_size);

typedef struct moe_ffn_plan {
    int64_t num_tokens, hidden_size, num_experts, top_k, intermediate_size;
    int32_t schedule;        /* 0 = weight-streaming (few rows per expert), 1 = LDS-tiled (many rows)    */
    int32_t permute_grid;    /* workgroups of each of the two permute kernels (count, scatter): one per    */
                             /* chunk of 1024 slots; 0 on the weight-streaming schedule, whose gate/up     */
                             /* kernel finds each expert's rows itself                                      */
    int32_t gateup_grid;     /* work tiles of the fused gate/up + SwiGLU grouped GEMM (upper bound on its */
                             /* workgroups: the streaming schedule runs a persistent grid of at most as    */
                             /* many workgroups as the GPU holds at once)                                  */
    int32_t down_grid;       /* work tiles of the down-projection grouped GEMM (same convention)           */
    int32_t block;           /* threads per workgroup of the GEMMs                                         */
    int32_t rows_per_tile;   /* token rows per GEMM tile                                                   */
    size_t workspace_bytes;  /* == moe_expert_ffn_workspace_bytes(...)                                    */
} moe_ffn_plan;
moe_status moe_expert_ffn_plan(int64_t num_tokens, int64_t hidden_size, int64_t num_experts, int64_t top_k,
                               int64_t intermediate_size, moe_ffn_plan* plan);

/* Kernel entry MoeExpertFFN(x, expertIds, weights, expertWeights, expertOut, workspace, tiling)
 * (op_kernel/moe_expert_ffn.cpp:613-621). */
moe_status moe_expert_ffn(const uint16_t* x, const int32_t* expert_ids, const uint16_t* weights,
                          const uint16_t* expert_weights, uint16_t* expert_out, void* workspace,
                          size_t workspace_bytes, int64_t num_tokens, int64_t hidden_size, int64_t num_experts,
                          int64_t top_k, int64_t intermediate_size, void* stream);

/* ------------------------------------------------------------------------------------------------------
 * MoeCombine: expert_out[T, K, H] fp16, expert_ids[T, K] int32 (not used by the math), weights[T, K] fp16
 *   -> y[T, H] fp16, y[t, :] = sum_k weights[t, k] * expert_out[t, k, :] accumulated in fp32 in ascending k
 *   (the reference kernel accumulates in fp16, op_kernel/moe_combine.cpp:87-106; its CPU references in fp32).
 *   Attr topK (default 2, op_host/moe_ops.cpp:665-667); K is taken from expert_out's dim 1.
 * ---------------------------------------------------------------------------------------------------- */

/* InferShape (op_host/moe_ops.cpp:495-515): y is [expert_out_dims[0], expert_out_dims[2]]. expert_ids_dims
 * may be NULL; when given it must be [T, K] (the TilingFunc rank check, op_host/moe_ops.cpp:425-428). */
moe_status moe_combine_infer_shape(const int64_t* expert_out_dims, int32_t expert_out_rank,
                                   const int64_t* expert_ids_dims, int32_t expert_ids_rank, int64_t y_dims[2]);
/* InferDataType (op_host/moe_ops.cpp:520-525): FLOAT16. */
moe_status moe_combine_infer_dtype(moe_dtype* y_dtype);

typedef struct moe_combine_plan {
    int64_t num_tokens, hidden_size, top_k;
    int32_t grid, block;
    int32_t elems_per_thread;
    size_t workspace_bytes; /* always 0 (op_host/moe_ops.cpp:477-481) */
} moe_combine_plan;
moe_status moe_combine_plan_for(int64_t num_tokens, int64_t hidden_size, int64_t top_k, moe_combine_plan* plan);

/* Kernel entry MoeCombine(expertOut, expertIds, weights, y, tiling) (op_kernel/moe_combine.cpp:136-143).
 * expert_ids may be NULL. */
moe_status moe_combine(const uint16_t* expert_out, const int32_t* expert_ids, const uint16_t* weights, uint16_t* y,
                       int64_t num_tokens, int64_t hidden_size, int64_t top_k, void* stream);

/* MoeExpertFFN that allocates nothing and takes no workspace. It has no counterpart in the reference. It is for
 * callers that cannot allocate device memory: code under HIP graph capture, tight serving loops, harnesses that
 * forbid hipMalloc.
 * The workspace is a fixed per-GPU device array inside the library (64 MiB, held by every GPU the library runs
 * on until the process ends). Sizes whose workspace exceeds it return MOE_ERR_UNSUPPORTED before anything is
 * launched (e.g. T*K*I*2 > ~60 MiB). The LDS-tiled schedule runs its down projection without the split
 * leftover round here, so expert_out can differ from moe_expert_ffn's in fp32 summation order on that schedule.
 * The weight-streaming schedule is bit-identical, except that an H above 2272 whose split gate/up partial sums
 * (splits x T*K x 2I x 4 bytes) do not fit runs gate/up unsplit (16-row passes, or the tiled schedule when H
 * exceeds 4568), with the same difference in summation order.
 * Every call on a GPU shares that GPU's array: calls that overlap on one GPU (two streams or threads) race.
 * The first call on each device looks up that device's array address and sets the kernels' LDS limits: make it
 * outside graph capture (one eager call per device); later calls may be captured and replayed.
 * Arguments, errors and outputs otherwise as moe_expert_ffn. */
moe_status moe_expert_ffn_no_alloc(const uint16_t* x, const int32_t* expert_ids, const uint16_t* weights,
                                   const uint16_t* expert_weights, uint16_t* expert_out, int64_t num_tokens,
                                   int64_t hidden_size, int64_t num_experts, int64_t top_k,
                                   int64_t intermediate_size, void* stream);

/* ------------------------------------------------------------------------------------------------------
 * Optional fast path: MoeExpertFFN followed by MoeCombine in one call. It has no single counterpart in the
 * reference; it chains the kernel entries MoeExpertFFN (op_kernel/moe_expert_ffn.cpp:613-621) and MoeCombine
 * (op_kernel/moe_combine.cpp:136-143), which stay the contract. expert_out is written exactly as
 * moe_expert_ffn writes it, and y is bit-identical to moe_combine(expert_out, expert_ids, weights, y, ...).
 * When the weight-streaming schedule splits the down projection over K, the split reduce produces y as well,
 * saving the combine pass over expert_out; otherwise the combine kernel runs after the FFN. Deterministic (no
 * global atomics). Workspace as for moe_expert_ffn. Sizes and errors as moe_expert_ffn plus moe_combine's checks.
 * ---------------------------------------------------------------------------------------------------- */
moe_status moe_expert_ffn_combine(const uint16_t* x, const int32_t* expert_ids, const uint16_t* weights,
                                  const uint16_t* expert_weights, uint16_t* expert_out, uint16_t* y,
                                  void* workspace, size_t workspace_bytes, int64_t num_tokens, int64_t hidden_size,
                                  int64_t num_experts, int64_t top_k, int64_t intermediate_size, void* stream);

/* ------------------------------------------------------------------------------------------------------
 * Optional fast path: the whole layer, MoeRoutingTopK -> MoeExpertFFN -> MoeCombine, in one call. It has no
 * single counterpart in the reference, whose harness chains the three operators (tests/test_moe.cpp:520-612:
 * routing, FFN, combine on one stream); the three operators stay the contract. On the LDS-tiled schedule the
 * routing kernel also ranks each token block's (token, k) slots by expert, so the FFN's permute is a single
 * scatter launch after it (the per-expert id scan of op_kernel/moe_expert_ffn.cpp:182-195, done once); on the
 * weight-streaming schedule it is routing (for T <= 16 and E > 64 spread over 4 * E / 32 workgroups, whose fp32
 * sums pass through the workspace) followed by moe_expert_ffn_combine. expert_ids, weights, expert_out and y are
 * bit-identical to the three calls'. Deterministic (no global atomics; nothing depends on timing).
 * The workspace is moe_layer_workspace_bytes() (>= moe_expert_ffn_workspace_bytes()); 0 = unsupported sizes.
 * Sizes and errors as the three operators' checks together.
 * ---------------------------------------------------------------------------------------------------- */
size_t moe_layer_workspace_bytes(int64_t num_tokens, int64_t hidden_size, int64_t num_experts, int64_t top_k,
                                 int64_t intermediate_size);
moe_status moe_layer(const uint16_t* x, const uint16_t* w_gate, const uint16_t* expert_weights,
                     int32_t* expert_ids, uint16_t* weights, uint16_t* expert_out, uint16_t* y, void* workspace,
                     size_t workspace_bytes, int64_t num_tokens, int64_t hidden_size, int64_t num_experts,
                     int64_t top_k, int64_t intermediate_size, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* MOE_OPS_H */
