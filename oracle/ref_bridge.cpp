// ref_bridge.cpp -- TEST INFRASTRUCTURE, NOT PRODUCT CODE.
//
// Builds the reference's own CPU simulator, tests/moe_cpu_sim.cpp, from the file where it lies under the
// reference checkout (oracle/Makefile passes -I<reference>/tests; nothing of it is copied into this
// repository), renames its main(), and exposes plain-pointer extern "C" wrappers around its functions so
// tests and bench.py can call the reference itself. The output goes only to oracle/_ref/.
//
// Wrapped reference functions (file:line in tests/moe_cpu_sim.cpp):
//   GenNormalData :161-167, NaiveMoE :183-306, ComputeRoutingTiling :68-93, TiledRouting :315-389,
//   ComputeExpertFFNTiling :99-123, TiledExpertFFN :395-494, ComputeCombineTiling :129-148,
//   TiledCombine :499-538, TiledMoE :543-569, CompareResults :586-604.

#define main moe_cpu_sim_reference_main
#include "moe_cpu_sim.cpp"
#undef main

#include <cstring>

namespace {
std::vector<float> as_vec(const float* p, size_t n) { return std::vector<float>(p, p + n); }
}  // namespace

extern "C" {

// The reference test's input generation (RunTest, tests/moe_cpu_sim.cpp:617-625): one mt19937(seed)
// stream feeds x [T,H], then w_gate [H,E], then expert_weights [E,3I,H], each N(0, 1/sqrt(H)).
void ref_gen_inputs(int T, int H, int E, int I, uint32_t seed, float* x, float* w_gate, float* ew) {
    std::mt19937 rng(seed);
    std::vector<float> vx, vg, vw;
    GenNormalData(vx, static_cast<size_t>(T) * H, H, rng);
    GenNormalData(vg, static_cast<size_t>(H) * E, H, rng);
    GenNormalData(vw, static_cast<size_t>(E) * 3 * I * H, H, rng);
    std::memcpy(x, vx.data(), vx.size() * sizeof(float));
    std::memcpy(w_gate, vg.data(), vg.size() * sizeof(float));
    std::memcpy(ew, vw.data(), vw.size() * sizeof(float));
}

// NaiveMoE: y [T,H].
void ref_naive_moe(const float* x, const float* w_gate, const float* ew, int T, int H, int E, int K, int I,
                   float* y) {
    std::vector<float> out;
    NaiveMoE(as_vec(x, static_cast<size_t>(T) * H), as_vec(w_gate, static_cast<size_t>(H) * E),
             as_vec(ew, static_cast<size_t>(E) * 3 * I * H), T, H, E, K, I, out);
    std::memcpy(y, out.data(), out.size() * sizeof(float));
}

// NaiveMoE on caller-owned vectors already holding the inputs; used by the CPU baseline so the timed region
// holds the reference computation only. Returns wall milliseconds measured around the NaiveMoE call.
double ref_naive_moe_timed(const float* x, const float* w_gate, const float* ew, int T, int H, int E, int K,
                           int I, float* y) {
    std::vector<float> vx = as_vec(x, static_cast<size_t>(T) * H);
    std::vector<float> vg = as_vec(w_gate, static_cast<size_t>(H) * E);
    std::vector<float> vw = as_vec(ew, static_cast<size_t>(E) * 3 * I * H);
    std::vector<float> out;
    auto t0 = std::chrono::high_resolution_clock::now();
    NaiveMoE(vx, vg, vw, T, H, E, K, I, out);
    auto t1 = std::chrono::high_resolution_clock::now();
    std::memcpy(y, out.data(), out.size() * sizeof(float));
    return std::chrono::duration<double, std::milli>(t1 - t0).count();
}

// TiledMoE: y [T,H]; returns wall milliseconds around the TiledMoE call.
double ref_tiled_moe_timed(const float* x, const float* w_gate, const float* ew, int T, int H, int E, int K,
                           int I, float* y) {
    std::vector<float> vx = as_vec(x, static_cast<size_t>(T) * H);
    std::vector<float> vg = as_vec(w_gate, static_cast<size_t>(H) * E);
    std::vector<float> vw = as_vec(ew, static_cast<size_t>(E) * 3 * I * H);
    std::vector<float> out;
    auto t0 = std::chrono::high_resolution_clock::now();
    TiledMoE(vx, vg, vw, T, H, E, K, I, out);
    auto t1 = std::chrono::high_resolution_clock::now();
    std::memcpy(y, out.data(), out.size() * sizeof(float));
    return std::chrono::duration<double, std::milli>(t1 - t0).count();
}

// TiledRouting (bit-identical to NaiveMoE steps 1-3): expert_ids [T,K] and weights [T,K].
void ref_routing(const float* x, const float* w_gate, int T, int H, int E, int K, int32_t* ids, float* weights) {
    auto tiling = ComputeRoutingTiling(T, H, E, K);
    std::vector<int> vid;
    std::vector<float> vw;
    TiledRouting(as_vec(x, static_cast<size_t>(T) * H), as_vec(w_gate, static_cast<size_t>(H) * E), T, H, E, K,
                 tiling, vid, vw);
    for (size_t i = 0; i < vid.size(); ++i) ids[i] = vid[i];
    std::memcpy(weights, vw.data(), vw.size() * sizeof(float));
}

// TiledExpertFFN: expert_out [T,K,H] for the given routing.
void ref_expert_ffn_tiled(const float* x, const float* ew, const int32_t* ids, const float* weights, int T, int H,
                          int E, int K, int I, float* expert_out) {
    auto tiling = ComputeExpertFFNTiling(T, H, I, E, K);
    std::vector<int> vid(ids, ids + static_cast<size_t>(T) * K);
    std::vector<float> out;
    TiledExpertFFN(as_vec(x, static_cast<size_t>(T) * H), as_vec(ew, static_cast<size_t>(E) * 3 * I * H), vid,
                   as_vec(weights, static_cast<size_t>(T) * K), T, H, E, K, I, tiling, out);
    std::memcpy(expert_out, out.data(), out.size() * sizeof(float));
}

// TiledCombine: y [T,H].
void ref_combine(const float* expert_out, const int32_t* ids, const float* weights, int T, int H, int K, float* y) {
    auto tiling = ComputeCombineTiling(T, H, K);
    std::vector<int> vid(ids, ids + static_cast<size_t>(T) * K);
    std::vector<float> out;
    TiledCombine(as_vec(expert_out, static_cast<size_t>(T) * K * H), vid, as_vec(weights, static_cast<size_t>(T) * K),
                 T, H, K, tiling, out);
    std::memcpy(y, out.data(), out.size() * sizeof(float));
}

// CompareResults: out = {maxAbsErr, meanAbsErr, cosSim}.
void ref_compare(const float* actual, const float* expected, int64_t n, double* out) {
    float mx = 0.0f, mean = 0.0f;
    double cs = 0.0;
    CompareResults(as_vec(actual, static_cast<size_t>(n)), as_vec(expected, static_cast<size_t>(n)), mx, mean, cs);
    out[0] = mx;
    out[1] = mean;
    out[2] = cs;
}

}  // extern "C"
