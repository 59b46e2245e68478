// Host-side fuzz driver for the C ABI (include/moe_ops.h), built with AddressSanitizer and UBSan on the host side
// of libmoe_mi355x.so. It launches no kernel: the launch calls get null pointers or a workspace one byte short,
// which their checks reject before any launch. It calls every entry point with seeded random and edge-case sizes
// (half of them drawn near valid shapes), ranks and attributes, and checks what the contract promises:
// statuses in range with an error message; InferShape outputs equal to the reference's rules; plans consistent
// with the workspace query; a workspace at least as large as the buffers it must hold (sorted slots, offsets, the
// fp16 intermediate [T*K, I]), so no size overflows into an under-sized buffer; the layer's workspace at least the
// FFN's; and launch calls that never report success for arguments they must reject.
// Usage: host_fuzz_abi ITERATIONS
#include <cinttypes>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <random>

#include "moe_ops.h"

namespace {

const int64_t kEdge[] = {-(int64_t{1} << 40), -2, -1, 0, 1, 2, 3, 7, 8, 13, 16, 31, 32, 33, 63, 64, 65, 96, 128, 200,
                         255, 256, 257, 1000, 1024, 1056, 1408, 2048, 4096, 7168, 8192, 14336, 16384, 65536,
                         1 << 20, (int64_t{1} << 31) - 1, int64_t{1} << 31, int64_t{1} << 32, int64_t{1} << 40,
                         INT64_MAX};
constexpr int kNumEdge = sizeof(kEdge) / sizeof(kEdge[0]);

int failures = 0;

#define CHECK(cond, ...)                                                   \
    do {                                                                   \
        if (!(cond)) {                                                     \
            if (failures < 20) {                                           \
                std::printf("FAIL line %d: %s | ", __LINE__, #cond);       \
                std::printf(__VA_ARGS__);                                  \
                std::printf("\n");                                         \
            }                                                              \
            ++failures;                                                    \
        }                                                                  \
    } while (0)

bool status_ok(moe_status st) { return st >= MOE_OK && st <= MOE_ERR_HIP; }

// A status other than MOE_OK must come with a message.
void check_status(moe_status st, const char* what) {
    CHECK(status_ok(st), "%s returned %d", what, static_cast<int>(st));
    if (st != MOE_OK) CHECK(std::strlen(moe_last_error()) > 0, "%s: empty error message", what);
}

// Exact product of non-negative sizes, or -1 when it does not fit in 63 bits.
int64_t mul(int64_t a, int64_t b) {
    if (a < 0 || b < 0) return -1;
    if (a != 0 && b > INT64_MAX / a) return -1;
    return a * b;
}

}  // namespace

int main(int argc, char** argv) {
    const long iters = argc > 1 ? std::atol(argv[1]) : 100000;
    std::mt19937_64 rng(20261202);
    auto pick = [&]() -> int64_t {
        if (rng() % 3 == 0) return static_cast<int64_t>(rng() % 20000) - 4;
        return kEdge[rng() % kNumEdge];
    };
    // fake device pointers for the launch calls: every call below fails a check before it could launch
    auto* fake = reinterpret_cast<uint16_t*>(uintptr_t{0x10000});
    auto* fake_i = reinterpret_cast<int32_t*>(uintptr_t{0x20000});
    long plans_ok = 0, ffn_ok = 0;
    for (long it = 0; it < iters; ++it) {
        int64_t T = pick(), H = pick(), E = pick(), K = pick(), I = pick();
        if (it % 2 == 1) {  // near valid shapes: the accepted paths of the planners
            H = 32 * static_cast<int64_t>(1 + rng() % 512);
            I = 32 * static_cast<int64_t>(1 + rng() % 1024);
            E = static_cast<int64_t>(1 + rng() % 256);
            K = static_cast<int64_t>(1 + rng() % (E < 16 ? E : 16));
            T = static_cast<int64_t>(rng() % 4 == 0 ? rng() % (int64_t{1} << 20) : rng() % 20000);
        }

        // ---- InferShape / InferDataType ----
        int64_t x_dims[3] = {T, H, pick()};
        const int32_t x_rank = rng() % 8 == 0 ? static_cast<int32_t>(rng() % 5) - 1 : 2;
        int64_t wg_dims[2] = {rng() % 4 ? H : pick(), E};
        int64_t ids_dims[2] = {-7, -7}, w_dims[2] = {-7, -7};
        moe_status st = moe_routing_topk_infer_shape(rng() % 50 ? x_dims : nullptr, x_rank, wg_dims, 2, K, ids_dims, w_dims);
        check_status(st, "moe_routing_topk_infer_shape");
        if (st == MOE_OK) {
            const int64_t k = K <= 0 ? 2 : K;
            CHECK(ids_dims[0] == T && ids_dims[1] == k && w_dims[0] == T && w_dims[1] == k,
                  "routing infer T=%" PRId64 " K=%" PRId64, T, K);
            CHECK(wg_dims[0] == H && x_rank == 2, "accepted H mismatch or rank %d", x_rank);
        }
        int64_t ew_dims[3] = {E, rng() % 4 ? mul(3, I) : pick(), rng() % 4 ? H : pick()};
        int64_t kid_dims[2] = {rng() % 4 ? T : pick(), K};
        int64_t out_dims[3] = {-7, -7, -7}, inter = -7;
        const int64_t attr = rng() % 4 ? 0 : pick();
        st = moe_expert_ffn_infer_shape(x_dims, 2, kid_dims, 2, ew_dims, 3, attr, out_dims, &inter);
        check_status(st, "moe_expert_ffn_infer_shape");
        if (st == MOE_OK) {
            CHECK(out_dims[0] == T && out_dims[1] == K && out_dims[2] == H, "ffn infer T=%" PRId64, T);
            // InferShape propagates shapes as the reference's does (op_host/moe_ops.cpp:363-386); sizes are
            // validated by the plan and the launch
            CHECK(ew_dims[1] % 3 == 0 && inter == ew_dims[1] / 3 && ew_dims[2] == H && kid_dims[0] == T,
                  "ffn infer inter=%" PRId64 " ew1=%" PRId64, inter, ew_dims[1]);
        }
        int64_t eo_dims[3] = {T, K, H}, y_dims[2] = {-7, -7};
        st = moe_combine_infer_shape(eo_dims, rng() % 8 ? 3 : 2, rng() % 3 ? kid_dims : nullptr, 2, y_dims);
        check_status(st, "moe_combine_infer_shape");
        if (st == MOE_OK) CHECK(y_dims[0] == T && y_dims[1] == H, "combine infer");

        // ---- plans and workspace sizes ----
        moe_routing_plan rp;
        st = moe_routing_topk_plan(T, H, E, K, &rp);
        check_status(st, "moe_routing_topk_plan");
        if (st == MOE_OK) {
            ++plans_ok;
            CHECK(rp.workspace_bytes == 0 && rp.block > 0 && rp.block <= 1024 && rp.lds_bytes >= 0 &&
                      rp.lds_bytes <= 160 * 1024 && rp.tokens_per_block > 0,
                  "routing plan T=%" PRId64 " H=%" PRId64 " E=%" PRId64, T, H, E);
            CHECK(mul(rp.grid, rp.tokens_per_block) >= T && (T == 0 || rp.grid > 0), "routing grid covers T");
        }
        moe_ffn_plan fp;
        st = moe_expert_ffn_plan(T, H, E, K, I, &fp);
        check_status(st, "moe_expert_ffn_plan");
        const size_t ws = moe_expert_ffn_workspace_bytes(T, H, E, K, I);
        const size_t lws = moe_layer_workspace_bytes(T, H, E, K, I);
        if (st == MOE_OK) {
            ++ffn_ok;
            CHECK(fp.workspace_bytes == ws, "plan ws %zu vs query %zu", fp.workspace_bytes, ws);
            CHECK(fp.schedule == 0 || fp.schedule == 1, "schedule %d", fp.schedule);
            const int64_t S = mul(T, K);
            const int64_t need = mul(S, mul(I, 2)) + mul(S, 4) + mul(E + 1, 4);  // hidden, sorted slots, offsets
            CHECK(S >= 0 && need >= 0 && static_cast<int64_t>(ws) >= need,
                  "workspace %zu below its buffers %" PRId64 " (T=%" PRId64 " H=%" PRId64 " E=%" PRId64
                  " K=%" PRId64 " I=%" PRId64 ")", ws, need, T, H, E, K, I);
            CHECK(lws >= ws, "layer workspace %zu below the FFN's %zu", lws, ws);
        } else {
            CHECK(ws == 0, "workspace %zu for sizes the plan rejects", ws);
        }
        moe_combine_plan cp;
        st = moe_combine_plan_for(T, H, K, &cp);
        check_status(st, "moe_combine_plan_for");
        if (st == MOE_OK) CHECK(cp.workspace_bytes == 0 && cp.block > 0, "combine plan");

        // ---- launches: null pointers, and fake pointers with a workspace one byte short ----
        st = moe_routing_topk(nullptr, fake, fake_i, fake, T, H, E, K, nullptr);
        check_status(st, "moe_routing_topk");
        CHECK(st != MOE_OK || T == 0, "routing accepted a null x");
        st = moe_expert_ffn(fake, fake_i, fake, fake, nullptr, fake, ws, T, H, E, K, I, nullptr);
        check_status(st, "moe_expert_ffn");
        CHECK(st != MOE_OK || T == 0, "ffn accepted a null expert_out");
        if (ws > 0) {
            st = moe_expert_ffn(fake, fake_i, fake, fake, fake, fake, ws - 1, T, H, E, K, I, nullptr);
            check_status(st, "moe_expert_ffn short workspace");
            CHECK(st != MOE_OK || T == 0, "ffn accepted a workspace one byte short");
        }
        st = moe_combine(fake, nullptr, fake, nullptr, T, H, K, nullptr);
        check_status(st, "moe_combine");
        CHECK(st != MOE_OK || T == 0, "combine accepted a null y");
        st = moe_expert_ffn_combine(fake, fake_i, fake, fake, fake, nullptr, fake, ws, T, H, E, K, I, nullptr);
        check_status(st, "moe_expert_ffn_combine");
        CHECK(st != MOE_OK || T == 0, "ffn_combine accepted a null y");
        if (lws > 0) {
            st = moe_layer(fake, fake, fake, fake_i, fake, fake, fake, fake, lws - 1, T, H, E, K, I, nullptr);
            check_status(st, "moe_layer short workspace");
            CHECK(st != MOE_OK || T == 0, "layer accepted a workspace one byte short");
        }
        st = moe_expert_ffn_no_alloc(fake, fake_i, fake, fake, nullptr, T, H, E, K, I, nullptr);
        check_status(st, "moe_expert_ffn_no_alloc");
        CHECK(st != MOE_OK || T == 0, "no_alloc accepted a null expert_out");
    }
    std::printf("%ld iterations, %ld routing plans and %ld FFN plans accepted, %d failures\n", iters, plans_ok, ffn_ok,
                failures);
    if (failures == 0) std::printf("ok\n");
    return failures == 0 ? 0 : 1;
}
