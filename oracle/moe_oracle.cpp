// moe_oracle.cpp -- TEST INFRASTRUCTURE, NOT PRODUCT CODE.
//
// A CPU restatement of the reference's fp32 MoE simulator, the checker for the HIP path. Only tests/,
// __graft_entry__.smoke() and bench.py's cpu_baseline leg may load the library built from this file; the
// product library never links or calls it.
//
// Reference followed: tests/moe_cpu_sim.cpp in Lu-Yu-Zhen/Implementing-MoE-Architecture-Operators-on-CANN-Platform
//   routing      NaiveMoE steps 1-3         tests/moe_cpu_sim.cpp:198-243  (also TiledRouting :315-389)
//   expert FFN   NaiveMoE step 4            tests/moe_cpu_sim.cpp:245-296
//                TiledExpertFFN             tests/moe_cpu_sim.cpp:395-494
//   combine      NaiveMoE step 5            tests/moe_cpu_sim.cpp:298-305  (also TiledCombine :499-538)
//   SiLU                                    tests/moe_cpu_sim.cpp:155-158
//   metric       CompareResults             tests/moe_cpu_sim.cpp:586-604  (here accumulated in double)
//
// Arithmetic contract, which is what makes these functions reproduce the reference bit for bit:
//   * Every dot product is a float accumulator that starts at 0.0f and adds float products in ascending
//     index order. Products and sums are rounded to fp32 separately: this file is compiled
//     `g++ -O2 -std=c++17` for baseline x86-64 (ISO mode => -ffp-contract=off, scalar SSE arithmetic),
//     exactly as build_cpu_sim.sh:19-23 compiles the reference.
//   * Softmax: max scan seeded with -1e30f, expf(l - max), sum in ascending expert order, then p / sum.
//   * Top-K: std::partial_sort of iota(E) with the comparator p[a] > p[b]. The same library routine is
//     called, so exact ties come out in the same (heap) order as the reference.
//   * Renormalisation: wSum accumulated over the K chosen experts in rank order, then w_k = p_k / wSum.
//   * Weight layout per expert e (tests/moe_cpu_sim.cpp:254-260):
//       W_gate[i][h] = ew[e*3*I*H +       i*H + h]    ([I, H] row-major)
//       W_up  [i][h] = ew[e*3*I*H + I*H + i*H + h]    ([I, H] row-major)
//       W_down[h][i] = ew[e*3*I*H + 2*I*H + h*I + i]  ([H, I] row-major)
//
// Pinning: tests/test_oracle.py checks every function here against the reference simulator compiled from
// its own source (oracle/_ref, bit-exact), against the committed golden vectors in tests/golden/, and
// against closed forms (one-hot inputs, K = 1 copies, softmax identities, brute-force fp64 GEMMs).

#include <algorithm>
#include <cmath>
#include <cstddef>
#include <cstdint>
#include <numeric>
#include <vector>

namespace {

inline float silu_ref(float v) { return v / (1.0f + expf(-v)); }

// Dot product of two float rows of length n with the reference's accumulation order.
inline float dot_seq(const float* a, const float* b, int64_t n) {
    float acc = 0.0f;
    for (int64_t j = 0; j < n; ++j) acc += a[j] * b[j];
    return acc;
}

bool dims_ok(int64_t T, int64_t H, int64_t E, int64_t K) {
    return T >= 0 && H > 0 && E > 0 && K >= 1 && K <= E;
}

// One token of routing: logits row -> (ids, weights) and the full softmax row.
void route_one(const float* logit, int64_t E, int64_t K, int32_t* ids, float* w, float* prob_row) {
    float mx = -1e30f;
    for (int64_t e = 0; e < E; ++e)
        if (logit[e] > mx) mx = logit[e];
    float total = 0.0f;
    for (int64_t e = 0; e < E; ++e) {
        prob_row[e] = expf(logit[e] - mx);
        total += prob_row[e];
    }
    for (int64_t e = 0; e < E; ++e) prob_row[e] /= total;

    std::vector<int> order(static_cast<size_t>(E));
    std::iota(order.begin(), order.end(), 0);
    std::partial_sort(order.begin(), order.begin() + K, order.end(),
                      [prob_row](int a, int b) { return prob_row[a] > prob_row[b]; });
    float sel = 0.0f;
    for (int64_t k = 0; k < K; ++k) {
        ids[k] = order[static_cast<size_t>(k)];
        sel += prob_row[order[static_cast<size_t>(k)]];
    }
    for (int64_t k = 0; k < K; ++k) w[k] = prob_row[order[static_cast<size_t>(k)]] / sel;
}

// SwiGLU expert FFN for one (token, slot): writes H outputs. `down_chunk` = 0 sums the down projection
// over the whole I range (naive schedule); > 0 sums per chunk of that many columns and adds the chunk
// partials in order (tiled schedule, tests/moe_cpu_sim.cpp:471-486).
void ffn_one(const float* xrow, const float* ew, int64_t e, int64_t H, int64_t I, int64_t down_chunk,
             float* out, std::vector<float>& hid) {
    const size_t base = static_cast<size_t>(e) * 3 * static_cast<size_t>(I) * static_cast<size_t>(H);
    const float* wg = ew + base;
    const float* wu = ew + base + static_cast<size_t>(I) * H;
    const float* wd = ew + base + 2 * static_cast<size_t>(I) * H;
    hid.resize(static_cast<size_t>(I));
    for (int64_t i = 0; i < I; ++i) {
        const float g = dot_seq(xrow, wg + static_cast<size_t>(i) * H, H);
        const float u = dot_seq(xrow, wu + static_cast<size_t>(i) * H, H);
        hid[static_cast<size_t>(i)] = silu_ref(g) * u;
    }
    for (int64_t h = 0; h < H; ++h) {
        const float* drow = wd + static_cast<size_t>(h) * I;
        if (down_chunk <= 0) {
            out[h] = dot_seq(hid.data(), drow, I);
        } else {
            float acc = 0.0f;
            for (int64_t c0 = 0; c0 < I; c0 += down_chunk) {
                const int64_t n = std::min<int64_t>(down_chunk, I - c0);
                acc += dot_seq(hid.data() + c0, drow + c0, n);
            }
            out[h] = acc;
        }
    }
}

}  // namespace

extern "C" {

// Routing for tokens [0, T): logits = x @ w_gate (w_gate is [H, E] row-major), softmax, top-K, K-renorm.
// probs_out / logits_out ([T, E]) may be null. Returns 0 on success, -1 on bad arguments.
int oracle_routing(const float* x, const float* w_gate, int64_t T, int64_t H, int64_t E, int64_t K,
                   int32_t* expert_ids, float* weights, float* probs_out, float* logits_out) {
    if (!x || !w_gate || !expert_ids || !weights || !dims_ok(T, H, E, K)) return -1;
    std::vector<float> logit(static_cast<size_t>(E)), prob(static_cast<size_t>(E));
    for (int64_t t = 0; t < T; ++t) {
        const float* xr = x + static_cast<size_t>(t) * H;
        for (int64_t e = 0; e < E; ++e) {
            float acc = 0.0f;
            for (int64_t h = 0; h < H; ++h) acc += xr[h] * w_gate[static_cast<size_t>(h) * E + e];
            logit[static_cast<size_t>(e)] = acc;
        }
        route_one(logit.data(), E, K, expert_ids + static_cast<size_t>(t) * K,
                  weights + static_cast<size_t>(t) * K, prob.data());
        if (probs_out) std::copy(prob.begin(), prob.end(), probs_out + static_cast<size_t>(t) * E);
        if (logits_out) std::copy(logit.begin(), logit.end(), logits_out + static_cast<size_t>(t) * E);
    }
    return 0;
}

// Expert FFN, naive schedule (token-major). Only tokens [t_begin, t_end) are computed; rows of other
// tokens in expert_out ([T, K, H]) are left untouched. Returns -1 on bad arguments or an id outside [0, E).
int oracle_expert_ffn(const float* x, const int32_t* expert_ids, const float* ew, int64_t T, int64_t H,
                      int64_t E, int64_t K, int64_t I, int64_t t_begin, int64_t t_end, float* expert_out) {
    if (!x || !expert_ids || !ew || !expert_out || !dims_ok(T, H, E, K) || I <= 0) return -1;
    if (t_begin < 0 || t_end > T || t_begin > t_end) return -1;
    std::vector<float> hid;
    for (int64_t t = t_begin; t < t_end; ++t)
        for (int64_t k = 0; k < K; ++k) {
            const int32_t e = expert_ids[static_cast<size_t>(t) * K + k];
            if (e < 0 || e >= E) return -1;
            ffn_one(x + static_cast<size_t>(t) * H, ew, e, H, I, 0,
                    expert_out + (static_cast<size_t>(t) * K + k) * H, hid);
        }
    return 0;
}

// Expert FFN, tiled schedule: experts in ascending order, each expert's (token, slot) pairs token-major,
// down projection summed per chunk of min(256, I) columns (tests/moe_cpu_sim.cpp:113,117,446-486).
int oracle_expert_ffn_tiled(const float* x, const int32_t* expert_ids, const float* ew, int64_t T, int64_t H,
                            int64_t E, int64_t K, int64_t I, float* expert_out) {
    if (!x || !expert_ids || !ew || !expert_out || !dims_ok(T, H, E, K) || I <= 0) return -1;
    for (int64_t s = 0; s < T * K; ++s)
        if (expert_ids[s] < 0 || expert_ids[s] >= E) return -1;
    const int64_t chunk = std::min<int64_t>(256, I);
    std::vector<float> hid;
    for (int64_t e = 0; e < E; ++e)
        for (int64_t t = 0; t < T; ++t)
            for (int64_t k = 0; k < K; ++k)
                if (expert_ids[static_cast<size_t>(t) * K + k] == e)
                    ffn_one(x + static_cast<size_t>(t) * H, ew, e, H, I, chunk,
                            expert_out + (static_cast<size_t>(t) * K + k) * H, hid);
    return 0;
}

// Combine: y[t, h] = sum_k weights[t, k] * expert_out[t, k, h], float accumulator from 0.0f, k ascending.
int oracle_combine(const float* expert_out, const float* weights, int64_t T, int64_t H, int64_t K, float* y) {
    if (!expert_out || !weights || !y || T < 0 || H <= 0 || K < 1) return -1;
    for (int64_t t = 0; t < T; ++t) {
        float* yr = y + static_cast<size_t>(t) * H;
        for (int64_t h = 0; h < H; ++h) yr[h] = 0.0f;
        for (int64_t k = 0; k < K; ++k) {
            const float w = weights[static_cast<size_t>(t) * K + k];
            const float* o = expert_out + (static_cast<size_t>(t) * K + k) * H;
            for (int64_t h = 0; h < H; ++h) yr[h] += w * o[h];
        }
    }
    return 0;
}

// Whole layer with the naive schedule (NaiveMoE, tests/moe_cpu_sim.cpp:183-306). Outputs other than y may
// be null. `tiled` != 0 uses the tiled FFN schedule instead (TiledMoE, tests/moe_cpu_sim.cpp:543-569).
int oracle_moe_layer(const float* x, const float* w_gate, const float* ew, int64_t T, int64_t H, int64_t E,
                     int64_t K, int64_t I, int tiled, int32_t* ids_out, float* weights_out, float* expert_out,
                     float* y) {
    if (!y || !dims_ok(T, H, E, K) || I <= 0) return -1;
    std::vector<int32_t> ids(static_cast<size_t>(T * K));
    std::vector<float> w(static_cast<size_t>(T * K));
    std::vector<float> eo(static_cast<size_t>(T * K * H), 0.0f);
    if (oracle_routing(x, w_gate, T, H, E, K, ids.data(), w.data(), nullptr, nullptr) != 0) return -1;
    const int rc = tiled ? oracle_expert_ffn_tiled(x, ids.data(), ew, T, H, E, K, I, eo.data())
                         : oracle_expert_ffn(x, ids.data(), ew, T, H, E, K, I, 0, T, eo.data());
    if (rc != 0) return -1;
    if (oracle_combine(eo.data(), w.data(), T, H, K, y) != 0) return -1;
    if (ids_out) std::copy(ids.begin(), ids.end(), ids_out);
    if (weights_out) std::copy(w.begin(), w.end(), weights_out);
    if (expert_out) std::copy(eo.begin(), eo.end(), expert_out);
    return 0;
}

// Accuracy metric: out = {max |a-b|, mean |a-b|, cosine(a, b)}, all accumulated in double. The reference
// accumulates the mean in float (tests/moe_cpu_sim.cpp:591,596); double removes that rounding.
void oracle_compare(const float* actual, const float* expected, int64_t n, double* out) {
    double mx = 0.0, sum = 0.0, ab = 0.0, aa = 0.0, bb = 0.0;
    for (int64_t i = 0; i < n; ++i) {
        const double a = actual[i], b = expected[i];
        const double d = std::fabs(a - b);
        sum += d;
        if (d > mx) mx = d;
        ab += a * b;
        aa += a * a;
        bb += b * b;
    }
    out[0] = mx;
    out[1] = n > 0 ? sum / static_cast<double>(n) : 0.0;
    out[2] = (aa > 0 && bb > 0) ? ab / (std::sqrt(aa) * std::sqrt(bb)) : 0.0;
}

}  // extern "C"
