// moe_routing.hip -- MoeRoutingTopK for gfx950.
//
// Reference: op_kernel/moe_routing.cpp (ComputeGate :238-254, SoftmaxRows :263-298, TopKSelect :304-369) and
// the CPU oracle NaiveMoE steps 1-3, tests/moe_cpu_sim.cpp:198-243.
//
// Narrow kernel, E <= 64: one workgroup owns 16 TB tokens (TB = 1, 2 or 4 blocks of 16, as many as keep >= 256
// workgroups, at most 2 for E > 32); W waves (16 when E <= 32, else 4, bounded by the LDS of the partials). Each
// w_gate fragment a wave builds is multiplied into all TB token blocks. The fragments come from w_gate rows staged
// in LDS and read back transposed (E % 8 == 0, 16-byte aligned w_gate), else from 8 strided 2-byte loads per
// lane; both give the same bits.
//   Phase 1: logits[16, E] = x[16, H] @ w_gate[H, E] on MFMA (v_mfma_f32_16x16x32_f16, fp32 accumulation;
//            fp16 x fp16 products are exact in fp32). The H/64 pairs of 32-wide k-steps are dealt round-robin to
//            the W waves (at decode and prefill, H = 2048 and W = 16: two pairs a wave), so each x load covers
//            whole 128-byte lines, re-laid through the wave's 2 KB x stage into the MFMA order; a wave issues the
//            loads of 1-2 pairs per round trip; it keeps partial logits of every expert block in registers and
//            parks them in LDS.
//   Fold:    one thread per (token, expert) adds the W partials in wave order.
//   Phase 2: one 16-lane DPP row per token for E <= 16, half a row (8 lanes) for larger E (each lane holding
//            Epad / 16 or Epad / 8 experts; 4 or 8 tokens per wave at a time) runs the softmax, top-K and
//            renormalisation with all-reduces over the token's lanes (select_row): max,
//            expf(l - max), sum, division by the sum; K rounds of an arg-max (lowest index wins an exact tie); the
//            renormalising sum over the K picks in rank order; fp16 round-to-nearest-even.
// From 32768 tokens, for 32 < E <= 64 and H = 1024 or 2048, the resident kernel replaces the narrow one with the
// same bits: one workgroup per CU holds the narrow kernel's w_gate fragments in registers and streams x through
// an LDS ring, so w_gate is read once per CU instead of once per 32 tokens.
// For E > 64 the rows kernel runs above 8192 tokens: a workgroup owns 64 tokens and each of its 4 waves 16 of them
// over all of H, so the selection runs on the accumulators. w_gate stages (16 KB, row-major) are copied into LDS
// with 16-byte direct-to-LDS loads and shared by the 4 waves; each wave's x rows stream through its own LDS ring
// 16 k-steps ahead. Up to 8192 tokens the quarters kernel runs: a workgroup owns 16 tokens and each of its 4 waves
// one quarter of H. Both add a token's H in the same four quarter sums, so the two give the same bits.
// T = 16384, H = 2048: E = 256, K = 8 75.8 us; E = 128 39.0 us (the wide kernel below: 171.7 and 95.1 us). When w_gate cannot be copied 16 bytes at a time (E % 8 != 0, unaligned) the wide
// kernel runs instead: its w_gate chunks are read with coalesced loads and written transposed, [expert][h], so a
// lane's B fragment is one ds_read_b128; a stage of 2-4 chunks is loaded into registers while the previous one is
// multiplied, two LDS buffers, one barrier per stage.
// HBM traffic per launch: T*H*2 (x) + H*E*2 (w_gate, L2-resident after the first workgroups) + T*K*6 bytes.

#include <type_traits>

#include "moe_device.h"
#include "moe_launch.h"
#include "moe_slot_rank.h"

namespace moe {

namespace {

constexpr int kTokensPerBlock = 16;
constexpr int kSelLanes = 16;  // lanes that select one token's experts (phase 2): one DPP row
// The narrow kernel's lanes per token: half a DPP row for E > 16. Fewer lanes per token each hold more experts,
// so the 64-bit arg-max steps cover twice the tokens per wave. DeepSeek shape (E = 64, K = 6): 20.7 against 21.6 us;
// at E = 16 (one expert per lane) 8 lanes were slower (decode 5.44 against 5.28 us); 4 lanes at E = 64 took 22.8 us.
constexpr int narrow_sel_lanes(int eb) { return eb == 1 ? 16 : 8; }

// The narrow kernel runs E <= 64. The wave count fixes each token's summation order (wave w adds the k-step pairs
// w, w + W, ..., each pair's two k-steps in order, and the partials are folded in wave order), so it does not
// depend on the token blocks: a token's ids and weights are the same whatever T is. 8 waves at E = 64 (two rounds
// of loads a wave instead of four) made DeepSeek routing slower: 30.6 against 26.8 us in the layer.
constexpr int waves_for(int eb, int /*tb*/) { return eb <= 2 ? 16 : 4; }
// k-steps whose loads are issued together (E <= 32 runs 1024 threads: 128 VGPRs per lane; E <= 64 256), for tb
// 16-token blocks per workgroup
constexpr int unroll_for(int eb, int tb) {
    return tb == 1 ? (eb == 1 ? 4 : eb == 2 ? 2 : 4) : eb == 1 ? (tb == 2 ? 4 : 2) : eb == 2 ? (tb == 2 ? 2 : 1) : 2;
}
// 16-token blocks per workgroup of the narrow kernel: each w_gate fragment a wave loads feeds tb of them. As many
// as keep the grid at >= 256 workgroups (one per CU), but at most 2 for 32 < E <= 64: two workgroups of 64 KB
// LDS then share a CU and one's selection phase overlaps the other's loads (T = 16384, E = 64: 22.8 us against
// 25.9 us with 4 blocks, 25.8 us with 1).
int narrow_token_blocks(int T, int eb) {
    const int tb = T >= 16 * 4 * 256 ? 4 : T >= 16 * 2 * 256 ? 2 : 1;
    return eb == 4 ? min(tb, 2) : tb;
}
// LW: k-steps per round trip (whole pairs), (TB + EB) * 4 VGPRs of loads each, within the 128 (1024 threads) or
// 256 (256 threads) a lane has
constexpr int lw_unroll(int tb) { return tb == 4 ? 2 : 4; }
// Each wave's 2 KB x stage (16 token rows x 128 B) lives in its own partial-logit rows when those hold 2 KB
// (16 TB tokens x 16 EB experts x 4 B), which phase 1 does not use yet; else it follows the w_gate stages.
constexpr bool narrow_xstage_in_part(int eb, int tb) { return tb * eb >= 2; }
// partial logits, then (lw) every wave's w_gate stage of 32 rows, then (one token and expert block) the x stages
constexpr size_t narrow_lds_bytes(int eb, int tb, bool lw) {
    return static_cast<size_t>(waves_for(eb, tb)) *
           (16 * eb * (tb * 16 * sizeof(float) + (lw ? 32 * sizeof(uint16_t) : 0)) +
            (narrow_xstage_in_part(eb, tb) ? 0 : 2048));
}
// the LDS path for w_gate: whole 16-byte chunks per row, an aligned base, 32-bit buffer offsets
bool narrow_lds_weights(const void* w_gate, int H, int E) {
    return E % 8 == 0 && (reinterpret_cast<uintptr_t>(w_gate) & 15) == 0 &&
           static_cast<int64_t>(H) * E * 2 < (int64_t{1} << 31);
}

// The 16-lane all-reduce runs on DPP row operations (a VALU operand modifier, no LDS round trip). Step 0 pairs
// lane i with i ^ 1 and step 1 with i ^ 2 (quad permutes); step 2 mirrors each half row (i <-> 7 - i, which
// pairs the two quads of the half, each already uniform) and step 3 the row (i <-> 15 - i, pairing the halves).
// Every lane ends with the row's result and the association is the same as a xor-1/2/4/8 butterfly's. Steps 0-2
// alone all-reduce each half row (8 lanes), like a xor-1/2/4 butterfly.
template <int STEP>
__device__ __forceinline__ int row_partner(int v) {
    constexpr int ctrl = STEP == 0 ? 0xB1 : STEP == 1 ? 0x4E : STEP == 2 ? 0x141 : 0x140;
    return __builtin_amdgcn_mov_dpp(v, ctrl, 0xF, 0xF, false);
}
template <int STEP>
__device__ __forceinline__ float row_partner(float v) {
    return __builtin_bit_cast(float, row_partner<STEP>(__builtin_bit_cast(int, v)));
}

// Softmax, top-K and renormalisation of one token per group of G lanes (a DPP row, G = 16, or half of one, G = 8;
// 64 / G tokens per wave); group lane gl holds experts gl + G q, q < EPL, of the token's logits row. The max and
// the arg-max (lowest index wins an exact tie, as the reference's strict '>' scans) are exact in any order; the
// softmax sum adds in one fixed association for a given G, identical in every lane of the group, so a token's
// result does not depend on its batch. Probabilities are exp(l - max) / sum, the K picks come in descending
// order, and their renormalisation sums them in rank order (the oracle's order, tests/moe_cpu_sim.cpp:224-243);
// lane gl writes picks gl, gl + G, ... below K. All 64 lanes of the wave must call this (DPP reads the
// neighbours' registers); only groups with `active` set write.
// select_vals takes the lane's logits v[q] (expert gl + G q) from registers; select_row reads them from an LDS
// row of the token's logits.
//
// The K rounds of arg-max over the 64-bit keys. Pick k sits in lane k % G, slot k / G of my_key; NP = 1 when
// K <= G (every lane holds at most one pick), else EPL (K <= E <= G EPL).
template <int EPL, int G, int NP>
__device__ __forceinline__ void pick_topk(uint64_t (&key)[EPL], int K, bool active, int32_t* ids_out,
                                          uint16_t* w_out) {
    const int gl = lane_id() & (G - 1);
    float sel = 0.0f;
    uint64_t my_key[NP];
#pragma unroll
    for (int j = 0; j < NP; ++j) my_key[j] = 0;
    for (int k = 0; k < K; ++k) {
        // the lane's own maximum as a pairwise tree (independent compares issue back to back)
        uint64_t tr[EPL];
#pragma unroll
        for (int q = 0; q < EPL; ++q) tr[q] = key[q];
#pragma unroll
        for (int w = 1; w < EPL; w *= 2)
#pragma unroll
            for (int q = 0; q + w < EPL; q += 2 * w) tr[q] = tr[q + w] > tr[q] ? tr[q + w] : tr[q];
        uint64_t best = tr[0];
#pragma unroll
        for (int st = 0; st < (G == 16 ? 4 : 3); ++st) {
            const uint32_t lo = static_cast<uint32_t>(best), hi = static_cast<uint32_t>(best >> 32);
            const uint32_t olo = static_cast<uint32_t>(st == 0   ? row_partner<0>(static_cast<int>(lo))
                                                       : st == 1 ? row_partner<1>(static_cast<int>(lo))
                                                       : st == 2 ? row_partner<2>(static_cast<int>(lo))
                                                                 : row_partner<3>(static_cast<int>(lo)));
            const uint32_t ohi = static_cast<uint32_t>(st == 0   ? row_partner<0>(static_cast<int>(hi))
                                                       : st == 1 ? row_partner<1>(static_cast<int>(hi))
                                                       : st == 2 ? row_partner<2>(static_cast<int>(hi))
                                                                 : row_partner<3>(static_cast<int>(hi)));
            const uint64_t other = (static_cast<uint64_t>(ohi) << 32) | olo;
            best = other > best ? other : best;
        }
#pragma unroll
        for (int q = 0; q < EPL; ++q)  // the index part alone is unique: exactly one lane owns the pick
            key[q] = static_cast<uint32_t>(key[q]) == static_cast<uint32_t>(best)
                         ? static_cast<uint64_t>(static_cast<uint32_t>(key[q]))
                         : key[q];
        if constexpr (NP == 1) {
            if ((k & (G - 1)) == gl) my_key[0] = best;
        } else {
#pragma unroll
            for (int j = 0; j < NP; ++j)
                if (k / G == j && (k & (G - 1)) == gl) my_key[j] = best;  // the first test is uniform
        }
        sel += __builtin_bit_cast(float, static_cast<uint32_t>(best >> 32) - 1u);
    }
    if (active) {
#pragma unroll
        for (int j = 0; j < NP; ++j) {
            if (gl + G * j < K) {
                ids_out[gl + G * j] = static_cast<int32_t>(~static_cast<uint32_t>(my_key[j]));
                const float pk = __builtin_bit_cast(float, static_cast<uint32_t>(my_key[j] >> 32) - 1u);
                w_out[gl + G * j] = f32_to_f16_bits(pk / sel);
            }
        }
    }
}

template <int EPL, int G = kSelLanes>
__device__ __forceinline__ void select_vals(float (&v)[EPL], int E, int K, bool active, int32_t* ids_out,
                                            uint16_t* w_out) {
    static_assert(G == 8 || G == 16, "a token's lanes: half a DPP row or a whole one");
    const int gl = lane_id() & (G - 1);
    float mx = -1e30f;  // the oracle's starting maximum
#pragma unroll
    for (int q = 0; q < EPL; ++q) {
        const int e = gl + G * q;
        v[q] = e < E ? v[q] : -1e30f;
        mx = fmaxf(mx, v[q]);
    }
    mx = fmaxf(mx, row_partner<0>(mx));
    mx = fmaxf(mx, row_partner<1>(mx));
    mx = fmaxf(mx, row_partner<2>(mx));
    if constexpr (G == 16) mx = fmaxf(mx, row_partner<3>(mx));
    float total = 0.0f;
#pragma unroll
    for (int q = 0; q < EPL; ++q) {
        v[q] = gl + G * q < E ? expf(v[q] - mx) : 0.0f;
        total += v[q];
    }
    total += row_partner<0>(total);
    total += row_partner<1>(total);
    total += row_partner<2>(total);
    if constexpr (G == 16) total += row_partner<3>(total);
    // One 64-bit key per candidate: the probability's bits + 1 above, the complemented expert index below. For
    // p >= 0 the bits order like the values, so the largest key is the largest probability and, among exact
    // ties, the lowest index (the reference's strict '>' scan in index order). Padding experts, NaN and picked
    // experts hold a zero upper word, below every candidate.
    uint64_t key[EPL];
#pragma unroll
    for (int q = 0; q < EPL; ++q) {
        const int e = gl + G * q;
        const float pq = v[q] / total;
        const uint32_t hi = e < E && pq == pq ? __builtin_bit_cast(uint32_t, pq) + 1u : 0u;  // NaN never wins
        key[q] = (static_cast<uint64_t>(hi) << 32) | static_cast<uint32_t>(~e);
    }
    if (K <= G)
        pick_topk<EPL, G, 1>(key, K, active, ids_out, w_out);
    else
        pick_topk<EPL, G, EPL>(key, K, active, ids_out, w_out);
}

template <int EPL, int G = kSelLanes>
__device__ __forceinline__ void select_row(const float* row, int E, int K, bool active, int32_t* ids_out,
                                           uint16_t* w_out) {
    const int gl = lane_id() & (G - 1);
    float v[EPL];
#pragma unroll
    for (int q = 0; q < EPL; ++q) v[q] = gl + G * q < E ? row[gl + G * q] : 0.0f;
    select_vals<EPL, G>(v, E, K, active, ids_out, w_out);
}

typedef short s16x4 __attribute__((ext_vector_type(4)));

// ds_read_b64_tr_b16 (gfx950): 8 bytes per lane, handed out transposed within each 16-lane group
__device__ __forceinline__ s16x4 lds_read_tr16(const uint8_t* p) {
    return __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) s16x4*)(p));
}

// LDS byte offset, inside a wave's w_gate stage ([32 rows][Epad] fp16, rows of 2 Epad 16-byte chunks), of the
// 16-byte chunk c of row r: chunks are XOR-swizzled by the row so that the transposing reads spread over the banks.
template <int EB>
__device__ __forceinline__ int wstage_chunk(int r, int c) {
    return (r * 2 * EB + (c ^ (r & (2 * EB - 1)))) * 16;
}

// EB = number of 16-expert blocks held in registers (ceil(E / 16) rounded up to an instantiated size); TB = 16-token
// blocks per workgroup (every w_gate fragment a wave loads is multiplied into all TB of them). LW: w_gate rows
// reach the wave through LDS (E % 8 == 0 and a 16-byte aligned w_gate): each k-step's 32 rows are loaded 16 bytes
// a lane and written to the wave's stage in their own row-major layout, and the B fragments (8 consecutive h of
// one expert) come out of ds_read_tr16_b64, which hands lane i of each 16-lane group element i % 4 of the
// 4-element rows addressed by lanes 4 j + i / 4 (j < 4). Without LW every fragment is 8 strided 2-byte global
// loads. NTX: x is loaded with the non-temporal hint (large batches, see kNtXBytes); the values are the same.
template <int EB, int TB, bool LW, bool NTX = false>
__global__ __launch_bounds__(waves_for(EB, TB) * kWave) void routing_topk_kernel(const uint16_t* __restrict__ x,
                                                                              const uint16_t* __restrict__ w_gate,
                                                                              int32_t* __restrict__ expert_ids,
                                                                              uint16_t* __restrict__ weights, int T,
                                                                              int H, int E, int K,
                                                                              int32_t* __restrict__ counts,
                                                                              int32_t* __restrict__ rank) {
    constexpr int W = waves_for(EB, TB);
    constexpr int Epad = EB * 16;
    constexpr int NT = 16 * TB;  // tokens per workgroup
    // [W][NT tokens][Epad] fp32 partial logits (row (0, t) receives the fold); with LW then [W][32][Epad] fp16
    extern __shared__ float part[];
    const int lane = lane_id();
    const int wave = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x) / kWave);  // uniform: scalar loops
    const int row = lane & 15;  // A row (token) / B column (expert) owned by this lane
    const int kg = lane >> 4;   // k-group: 8 consecutive k of each 32-wide k-step
    const int t0 = static_cast<int>(blockIdx.x) * NT;

    // ---- phase 1: partial logits on MFMA ----
    // x arrives in whole 128-byte lines: wave w owns the k-step pairs P = w, w + W, ... (k-steps 2P, 2P + 1, i.e.
    // 64 columns = one line of each token row), and a load instruction covers 8 token rows x 128 B (lane -> row
    // lane / 8 + 8 h, 16-byte chunk lane % 8). The wave re-lays each 16-row block through 2 KB of LDS (its own
    // x stage: 128-byte rows, chunk c of row r at c ^ ((r >> 1) & 7)) into the MFMA A order (row, k-group). Half-line
    // loads straight into that order (16 rows x 64 B per instruction) held a CU's outstanding requests to half the
    // bytes: 32 MB of x took ~11 us more than no x at all, against 6.6 us for a streaming read of the same bytes.
    const int xr = lane >> 3, xc = lane & 7;  // line loads: row (+ 8 h) and chunk of this lane
    const uint16_t* xline[TB][2];
#pragma unroll
    for (int tb = 0; tb < TB; ++tb)
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const int tok = min(t0 + tb * 16 + xr + 8 * h, T - 1);  // rows past T read a valid row; results dropped
            xline[tb][h] = x + static_cast<size_t>(tok) * H + xc * 8;
        }
    f32x4 acc[TB][EB];
#pragma unroll
    for (int tb = 0; tb < TB; ++tb)
#pragma unroll
        for (int b = 0; b < EB; ++b) acc[tb][b] = f32x4{0.f, 0.f, 0.f, 0.f};

    const int nsteps = H / 32;
    const int npairs = (nsteps + 1) / 2;  // an odd nsteps leaves the last pair's second k-step empty
    // this wave's x stage: its own partial-logit rows (unused until phase 1 ends) when they hold 2 KB, else a
    // region after the w_gate stages
    uint8_t* xst = narrow_xstage_in_part(EB, TB)
                       ? reinterpret_cast<uint8_t*>(part + wave * NT * Epad)
                       : reinterpret_cast<uint8_t*>(part + W * NT * Epad) + (LW ? W * 32 * Epad * 2 : 0) + wave * 2048;
    const int swr = (row >> 1) & 7;  // the A-fragment reads' swizzle (row = the lane's 16-row block row)
    // x of pair P (column 64 P) into registers: 2 line loads per token block; the second k-step's chunks of a pair
    // whose second k-step is past H read the first k-step's columns instead (in bounds) and are dropped below
    auto load_x = [&](f16x8 (&xl)[TB][2], int P) __attribute__((always_inline)) {
        const int col = P * 64 - (xc >= 4 && 2 * P + 1 >= nsteps ? 32 : 0);
#pragma unroll
        for (int tb = 0; tb < TB; ++tb)
#pragma unroll
            for (int h = 0; h < 2; ++h) xl[tb][h] = NTX ? load_f16x8_stream(xline[tb][h] + col) : load_f16x8(xline[tb][h] + col);
    };
    // the A fragments of both k-steps of the pair, per token block, through the x stage (zeros for a k-step past
    // H, whatever x holds: 0 * inf would be NaN)
    auto relayout_x = [&](const f16x8 (&xl)[TB][2], f16x8 (&a)[TB][2], bool in1) __attribute__((always_inline)) {
#pragma unroll
        for (int tb = 0; tb < TB; ++tb) {
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                const int r = xr + 8 * h;
                *reinterpret_cast<f16x8*>(xst + r * 128 + ((xc ^ ((r >> 1) & 7)) << 4)) = xl[tb][h];
            }
            // the reads take what other lanes of this wave just wrote (LDS operations of one wave run in order)
            __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
            __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
#pragma unroll
            for (int st = 0; st < 2; ++st)
                a[tb][st] = *reinterpret_cast<const f16x8*>(xst + row * 128 + (((4 * st + kg) ^ swr) << 4));
            __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");  // read before the next block's writes
            __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
            if (!in1) a[tb][1] = f16x8{};
        }
    };
    // LW: this wave's stage, and each lane's chunk and fragment offsets
    uint8_t* wst = reinterpret_cast<uint8_t*>(part + W * NT * Epad) + wave * (32 * Epad * 2);
    int cpy_off[EB];     // byte offset in w_gate (relative to the k-step's first row) of the chunk this lane copies
    int frag_off[2][EB]; // byte offset in a stage of the 8 bytes this lane addresses for half h of expert block b
    if constexpr (LW) {
#pragma unroll
        for (int i = 0; i < EB; ++i) {  // copy i fills stage bytes [1024 i, 1024 i + 1024): lane -> 16-byte slot
            const int slot = i * kWave + lane;
            const int r = slot / (2 * EB), pc = slot % (2 * EB);
            const int c = pc ^ (r & (2 * EB - 1));     // the logical chunk that belongs in physical slot pc
            cpy_off[i] = (r * E + (c * 8 < E ? c * 8 : 0)) * 2;  // padding chunks copy any valid chunk
        }
        const int g = lane >> 4, sl = lane & 15;
#pragma unroll
        for (int h = 0; h < 2; ++h)
#pragma unroll
            for (int b = 0; b < EB; ++b) {
                const int r = 8 * g + 4 * h + sl / 4;
                const int e = 16 * b + 4 * (sl % 4);
                frag_off[h][b] = wstage_chunk<EB>(r, e / 8) + (e % 8) * 2;
            }
    }
    if constexpr (LW) {
        // UP pairs per round trip: their x lines and w_gate chunks are all loaded into registers first (16 bytes a
        // lane each), then pair by pair the x lines are re-laid into A fragments and k-step by k-step the w_gate
        // chunks are written to the wave's LDS stage (row-major, XOR-swizzled 16-byte chunks), read back as B
        // fragments by ds_read_tr16_b64 and multiplied. The k-steps add in the order 2 p0, 2 p0 + 1, 2 (p0 + W),
        // ... (Direct-to-LDS copies of the chunks were used here before: the compiler waits for every copy in
        // flight before any LDS read, which held a round trip to 2 k-steps.)
        constexpr int UP = lw_unroll(TB) / 2;
        const uint8_t* wbytes = reinterpret_cast<const uint8_t*>(w_gate);
        // FULL: all UP pairs of the round exist; the last round of a wave may run past H, and its extra pairs
        // load pair 0 and multiply zeros (every step runs, so no load is moved behind a branch)
        auto round = [&](int p0, auto full) __attribute__((always_inline)) {
            constexpr bool FULL = decltype(full)::value;
            f16x8 xl[UP][TB][2];
            u32x4 wv[UP][2][EB];
#pragma unroll
            for (int v = 0; v < UP; ++v) {
                const int P = p0 + v * W;
                const int Pc = FULL || P < npairs ? P : 0;
                load_x(xl[v], Pc);
#pragma unroll
                for (int st = 0; st < 2; ++st) {
                    const int k0 = min(2 * Pc + st, nsteps - 1) * 32;
#pragma unroll
                    for (int i = 0; i < EB; ++i)
                        wv[v][st][i] = *reinterpret_cast<const u32x4*>(wbytes + static_cast<size_t>(k0) * E * 2 + cpy_off[i]);
                }
            }
            __builtin_amdgcn_sched_barrier(0);  // all UP pairs' loads are issued before the first is waited for
#pragma unroll
            for (int v = 0; v < UP; ++v) {
                const int P = p0 + v * W;
                const bool in0 = FULL || P < npairs, in1 = in0 && 2 * P + 1 < nsteps;
                f16x8 a[TB][2];
                relayout_x(xl[v], a, in1);
                if (!in0) {  // a pair past H contributes nothing, whatever x holds
#pragma unroll
                    for (int tb = 0; tb < TB; ++tb) a[tb][0] = f16x8{};
                }
#pragma unroll
                for (int st = 0; st < 2; ++st) {
                    const bool in = st == 0 ? in0 : in1;
#pragma unroll
                    for (int i = 0; i < EB; ++i) *reinterpret_cast<u32x4*>(wst + i * 1024 + lane * 16) = wv[v][st][i];
                    f16x8 bv[EB];
#pragma unroll
                    for (int b = 0; b < EB; ++b) {
                        const s16x4 lo = lds_read_tr16(wst + frag_off[0][b]);
                        const s16x4 hi = lds_read_tr16(wst + frag_off[1][b]);
                        bv[b] = in ? __builtin_bit_cast(f16x8, __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7))
                                   : f16x8{};
                    }
#pragma unroll
                    for (int tb = 0; tb < TB; ++tb)
#pragma unroll
                        for (int b = 0; b < EB; ++b) acc[tb][b] = mfma16x16x32(a[tb][st], bv[b], acc[tb][b]);
                }
            }
        };
        int p0 = wave;
        for (; p0 + (UP - 1) * W < npairs; p0 += UP * W) round(p0, std::true_type{});
        if (p0 < npairs) round(p0, std::false_type{});
    } else {  // w_gate B fragments as 8 strided 2-byte loads each, UP pairs per round trip
        constexpr int UP = unroll_for(EB, TB) >= 2 ? unroll_for(EB, TB) / 2 : 1;
        for (int p0 = wave; p0 < npairs; p0 += UP * W) {
            f16x8 xl[UP][TB][2];
            f16x8 bv[UP][2][EB];
#pragma unroll
            for (int v = 0; v < UP; ++v) {
                const int P = p0 + v * W;
                const int Pc = P < npairs ? P : 0;
                load_x(xl[v], Pc);
#pragma unroll
                for (int st = 0; st < 2; ++st) {
                    const bool in = P < npairs && 2 * P + st < nsteps;
                    const uint16_t* wrow = w_gate + static_cast<size_t>(min(2 * Pc + st, nsteps - 1) * 32 + kg * 8) * E;
#pragma unroll
                    for (int b = 0; b < EB; ++b) {
                        const int e = b * 16 + row;
#pragma unroll
                        for (int q = 0; q < 8; ++q)
                            bv[v][st][b][q] = (in && e < E) ? __builtin_bit_cast(f16, wrow[static_cast<size_t>(q) * E + e])
                                                            : static_cast<f16>(0.0f);
                    }
                }
            }
#pragma unroll
            for (int v = 0; v < UP; ++v) {
                const int P = p0 + v * W;
                f16x8 a[TB][2];
                relayout_x(xl[v], a, P < npairs && 2 * P + 1 < nsteps);
                if (!(P < npairs)) {  // a pair past H contributes nothing, whatever x holds
#pragma unroll
                    for (int tb = 0; tb < TB; ++tb) a[tb][0] = f16x8{};
                }
#pragma unroll
                for (int st = 0; st < 2; ++st)
#pragma unroll
                    for (int tb = 0; tb < TB; ++tb)
#pragma unroll
                        for (int b = 0; b < EB; ++b) acc[tb][b] = mfma16x16x32(a[tb][st], bv[v][st][b], acc[tb][b]);
            }
        }
    }
    // the x stage may be this wave's partial-logit rows: every stage read is done before they are written
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    // D[token tb*16 + 4*kg + r][expert b*16 + row]
#pragma unroll
    for (int tb = 0; tb < TB; ++tb)
#pragma unroll
        for (int b = 0; b < EB; ++b)
#pragma unroll
            for (int r = 0; r < 4; ++r) part[(wave * NT + tb * 16 + kg * 4 + r) * Epad + b * 16 + row] = acc[tb][b][r];
    __syncthreads();

    // ---- fold: partial of wave 0 + wave 1 + ... in wave order, into the wave-0 rows ----
    f32x4* part4 = reinterpret_cast<f32x4*>(part);
    for (int i = static_cast<int>(threadIdx.x); i < NT * Epad / 4; i += W * kWave) {
        f32x4 v = part4[i];
#pragma unroll
        for (int w = 1; w < W; ++w) v += part4[w * NT * Epad / 4 + i];
        part4[i] = v;
    }
    __syncthreads();

    // ---- phase 2: G lanes per token (Epad / G experts a lane), 64 / G tokens per wave at a time ----
    constexpr int G = narrow_sel_lanes(EB);
    constexpr int TPW = kWave / G;  // tokens per wave and round
    for (int tb = wave * TPW; tb < NT; tb += W * TPW) {
        const int t = tb + lane / G;
        const bool active = t < NT && t0 + t < T;
        const int tr = min(t, NT - 1);  // inactive groups read a valid row and write nothing
        select_row<Epad / G, G>(part + tr * Epad, E, K, active, expert_ids + static_cast<size_t>(t0 + tr) * K,
                       weights + static_cast<size_t>(t0 + tr) * K);
    }
    // ---- optional tail: the block's slots ranked by expert, for the permute's scatter ----
    if (counts != nullptr) {
        __syncthreads();  // the block's ids are written and part[] is no longer read
        constexpr int MAXIT = (NT * kRankTopK + W * kWave - 1) / (W * kWave);
        rank_slots<W, MAXIT>(expert_ids, t0 * K, min(T, t0 + NT) * K, E, counts_stride(E),
                             reinterpret_cast<int*>(part), counts + static_cast<size_t>(blockIdx.x) * counts_stride(E),
                             rank);
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
                                                                           int H, int E, int K,
                                                                           int32_t* __restrict__ counts,
                                                                           int32_t* __restrict__ rank) {
    constexpr int Epad = EB * 16;
    constexpr int CH = wide_chunks(EB);
    constexpr int P = wide_pitch(EB);
    constexpr int kThreads = kWideWaves * kWave;
    constexpr int kPer = (CH * 32 * Epad + kThreads - 1) / kThreads;  // w_gate elements per thread per stage
    extern __shared__ __align__(16) uint16_t wt[];                   // [2][Epad][P] halfs, then logits
    float* logits = reinterpret_cast<float*>(wt + 2 * Epad * P);     // [64 tokens][Epad] fp32
    const int tid = static_cast<int>(threadIdx.x);
    const int lane = lane_id();
    const int wave = __builtin_amdgcn_readfirstlane(tid / kWave);
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

    // ---- 16 lanes per token (EB experts a lane), 4 tokens per wave at a time ----
    constexpr int TPW = kWave / kSelLanes;
    for (int tb = wave * TPW; tb < kWideTokens; tb += kWideWaves * TPW) {
        const int t = tb + lane / kSelLanes;
        const bool active = t0 + t < T;
        select_row<EB>(logits + t * Epad, E, K, active, expert_ids + static_cast<size_t>(active ? t0 + t : 0) * K,
                       weights + static_cast<size_t>(active ? t0 + t : 0) * K);
    }
    // ---- optional tail: the block's slots ranked by expert, for the permute's scatter ----
    if (counts != nullptr) {
        __syncthreads();  // the block's ids are written and the logits are no longer read
        constexpr int MAXIT = (kWideTokens * kRankTopK + kWideWaves * kWave - 1) / (kWideWaves * kWave);
        rank_slots<kWideWaves, MAXIT>(expert_ids, t0 * K, min(T, t0 + kWideTokens) * K, E, counts_stride(E),
                                      reinterpret_cast<int*>(logits),
                                      counts + static_cast<size_t>(blockIdx.x) * counts_stride(E), rank);
    }
}

// ---- the rows kernel: each wave owns 16 tokens over all of H, w_gate stages shared by the workgroup ----
// A workgroup of kRowWaves waves routes kRowTokens tokens. Per stage of SK 32-row k-steps (16 KB of w_gate):
//   * the four waves copy the stage's w_gate rows, in their own row-major layout (16-byte chunks XOR-swizzled by
//     row), into a ring of kRowWStages shared LDS stages with 16-byte direct-to-LDS loads, three stages ahead,
//     one barrier per stage;
//   * each wave copies its 16 token rows of x (64 B per row and k-step) into its own LDS ring, kRowXDepth k-steps
//     ahead of their use, so each CU keeps ~64 KB of x in flight without spending registers on it;
//   * A fragments are ds_read_b128 from the x ring, B fragments two ds_read_b64_tr_b16 from the w_gate stage.
// The k-steps of each quarter of H add in order (quarter_begin below). The kernel runs for E > 64 whenever its
// copies can (E % 8 == 0, a 16-byte aligned w_gate, SK dividing H / 32) and T > 8192; the quarters kernel gives
// the same bits below that, so a token's bits do not depend on its batch.
// At E <= 64 it was slower than the narrow kernel (T = 16384, E = 64: 27.8 µs alone and 34.2 µs in the layer,
// against 21.8 and 30.2 µs): every wave reads all of w_gate from LDS, four times the narrow kernel's share.
// At few tokens each 16-token block multiplies all of w_gate on one CU, and the compiler's wait for every copy in
// flight before a transposing read (see the quarters kernel) leaves the ring no deeper than one stage, so the time
// does not fall with T: H = 7168, E = 256 (3.7 MB of w_gate) 140 µs at T = 1, 185 µs at T = 128 to 2048, where
// the quarters kernel takes 44-55 µs. Measured before it and not kept: workgroups of 1 or 2 waves (16 or 32
// tokens, more CUs) 137 / 145 µs at T = 128 but 385 / 362 µs at T = 16384; a 7-stage w_gate ring 187 µs; the
// rows kernel double-buffered with each stage read whole before the next one's copies, as the quarters kernel
// does, 192 µs at T = 128 and 2x slower at E = 128.
// The selection then runs on the accumulators: the MFMA leaves lane (row kg = lane / 16, column n) with token
// 4 kg + r, expert 16 b + n in acc[b][r], i.e. each 16-lane DPP row holds one token's experts as select_vals
// wants them.
// The H reduction of the rows and quarters kernels: the stages fall into four quarters (quarter j = stages
// [j nst / 4, (j + 1) nst / 4)), each summed in k order from zero, and the quarter sums are added as
// ((q0 + q1) + q2) + q3. The rows kernel sums the quarters one after the other in each wave; the quarters kernel
// gives each quarter to a wave of its own. Both make the same fp32 operations for a token, so its logits, ids and
// weights do not depend on which of them ran.
__host__ __device__ __forceinline__ int quarter_begin(int j, int nst) { return j * nst / 4; }

constexpr int kRowWaves = 4;
constexpr int kRowTokens = 16 * kRowWaves;
constexpr int kRowXDepth = 16;                                               // x k-steps in flight per wave
constexpr int kRowWStages = 4;                                               // w_gate ring: 3 stages ahead
constexpr int row_stage_ksteps(int eb) { return eb >= 16 ? 1 : 16 / eb; }   // 16 KB of w_gate per stage
constexpr size_t row_lds_bytes(int eb) {
    return kRowWStages * 16384 + static_cast<size_t>(kRowWaves) * (kRowXDepth + row_stage_ksteps(eb)) * 1024;
}

template <int EB>
__global__ __launch_bounds__(kRowWaves * kWave) void routing_rows_kernel(const uint16_t* __restrict__ x,
                                                                          const uint16_t* __restrict__ w_gate,
                                                                          int32_t* __restrict__ expert_ids,
                                                                          uint16_t* __restrict__ weights, int T,
                                                                          int H, int E, int K,
                                                                          int32_t* __restrict__ counts,
                                                                          int32_t* __restrict__ rank) {
    constexpr int Epad = EB * 16;
    constexpr int SK = row_stage_ksteps(EB);
    constexpr int NW = kRowWStages;       // w_gate ring slots; stage i + NW - 1 is copied while i is used
    constexpr int NXS = kRowXDepth / SK;  // x stages issued ahead of the one in use (>= NW, see the wait below)
    constexpr int XR = NXS + 1;           // x ring slots (stages) per wave
    constexpr int kStage = SK * 32 * Epad * 2;
    static_assert(kStage == 16384 && NXS >= NW && NW >= 2, "stage geometry");
    extern __shared__ __align__(16) uint8_t lds[];
    const int lane = lane_id();
    const int wave = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x) / kWave);
    uint8_t* wbuf = lds;                                          // [NW][kStage]
    uint8_t* xbuf = lds + NW * kStage + wave * XR * SK * 1024;    // this wave's ring: [XR][SK][16 rows][64 B]
    const int t0 = static_cast<int>(blockIdx.x) * kRowTokens;
    const int nst = H / 32 / SK;  // the host runs this kernel only when SK divides H / 32

    const __amdgpu_buffer_rsrc_t wrs =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t*>(w_gate), 0, H * E * 2, 0x00020000);
    // x rows of this workgroup's tokens only (at most kRowTokens rows: 32-bit offsets for any T)
    const __amdgpu_buffer_rsrc_t xrs = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<uint16_t*>(x + static_cast<size_t>(t0) * H), 0, min(kRowTokens, T - t0) * H * 2, 0x00020000);
    // x copy: lane -> row lane / 4 (token t0 + 16 wave + row, clamped into the batch), 16-byte chunk lane % 4
    const int xoff = (min(wave * 16 + lane / 4, T - 1 - t0) * H + (lane % 4) * 8) * 2;
    // w_gate copy: wave w fills 1 KB slabs w, w + 4, w + 8, w + 12 of a stage; lane -> 16-byte slot of the slab
    int woff[4];
#pragma unroll
    for (int m = 0; m < 4; ++m) {
        const int off = (wave + 4 * m) * 1024 + lane * 16;
        const int R = off / (32 * EB), pc = (off % (32 * EB)) / 16;  // stage row (SK k-steps of 32), slot
        const int c = pc ^ ((R % 32) & (2 * EB - 1));                 // the logical chunk stored in slot pc
        woff[m] = (R * E + (c * 8 < E ? c * 8 : 0)) * 2;              // padding chunks copy any valid chunk
    }
    // fragment reads: A at row * 64 + kg * 16 of a k-step's x block; B as in the narrow kernel's LDS path
    const int arow = lane & 15, kg = lane >> 4;
    int frag_off[2][EB];
    {
        const int sl = lane & 15;
#pragma unroll
        for (int h = 0; h < 2; ++h)
#pragma unroll
            for (int b = 0; b < EB; ++b) {
                const int r = 8 * kg + 4 * h + sl / 4;
                const int e = 16 * b + 4 * (sl % 4);
                frag_off[h][b] = wstage_chunk<EB>(r, e / 8) + (e % 8) * 2;
            }
    }
    auto issue_w = [&](int st) __attribute__((always_inline)) {
        uint8_t* dst = wbuf + (st % NW) * kStage;
#pragma unroll
        for (int m = 0; m < 4; ++m)
            __builtin_amdgcn_raw_ptr_buffer_load_lds(wrs, (__attribute__((address_space(3))) void*)(dst + (wave + 4 * m) * 1024),
                                                     16, static_cast<int>(woff[m]), st * SK * 32 * E * 2, 0, 0);
    };
    auto issue_x = [&](int st) __attribute__((always_inline)) {
#pragma unroll
        for (int ks = 0; ks < SK; ++ks)
            __builtin_amdgcn_raw_ptr_buffer_load_lds(xrs, (__attribute__((address_space(3))) void*)(xbuf + ((st % XR) * SK + ks) * 1024),
                                                     16, xoff, (st * SK + ks) * 64, 0, 0);
    };

    f32x4 acc[EB];   // the current quarter's sum
    f32x4 qsum[EB];  // the finished quarters' sum, ((q0 + q1) + q2)
#pragma unroll
    for (int b = 0; b < EB; ++b) acc[b] = qsum[b] = f32x4{0.f, 0.f, 0.f, 0.f};

    // Issue order: x(0 .. NXS-1), w(0 .. NW-2), then per iteration j: w(j + NW - 1), x(j + NXS).
    for (int st = 0; st < min(NXS, nst); ++st) issue_x(st);
    for (int st = 0; st < min(NW - 1, nst); ++st) issue_w(st);
    // The quarters run one after the other (the copies run on across their boundaries); each starts from zero and
    // joins the sum when it ends.
    int i = 0;
    for (int j = 0; j < 4; ++j) {
        for (const int iend = quarter_begin(j + 1, nst); i < iend; ++i) {
            // This wave's copies of w_gate stage i and of x stage i have landed. After w(i) (iteration i - NW + 1, or
            // the prologue) came x(i - NW + 1 + NXS) and then NW - 2 iterations of w + x: SK + (NW - 2)(4 + SK) copies
            // when every one of them went out, i.e. when iteration i - 1 still issued both; otherwise wait for all.
            // x(i) went out no later than iteration i - NXS <= i - NW, before w(i).
            if (i >= NW - 1 && i + NW - 2 < nst && i - 1 + NXS < nst) {
                __builtin_amdgcn_s_waitcnt(vmcnt_imm(SK + (NW - 2) * (4 + SK)));
            } else {
                __builtin_amdgcn_s_waitcnt(vmcnt_imm(0));
            }
            __syncthreads();  // every wave's w(i) is visible; every wave is done with w(i - 1) and its x(i - 1)
            if (i + NW - 1 < nst) issue_w(i + NW - 1);
            if (i + NXS < nst) issue_x(i + NXS);
            const uint8_t* ws = wbuf + (i % NW) * kStage;
            const uint8_t* xs = xbuf + (i % XR) * SK * 1024;
#pragma unroll
            for (int ks = 0; ks < SK; ++ks) {
                const f16x8 a = *reinterpret_cast<const f16x8*>(xs + ks * 1024 + arow * 64 + kg * 16);
                const uint8_t* wk = ws + ks * 32 * Epad * 2;
#pragma unroll
                for (int b = 0; b < EB; ++b) {
                    const s16x4 lo = lds_read_tr16(wk + frag_off[0][b]);
                    const s16x4 hi = lds_read_tr16(wk + frag_off[1][b]);
                    const f16x8 bv = __builtin_bit_cast(f16x8, __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7));
                    acc[b] = mfma16x16x32(a, bv, acc[b]);
                }
            }
        }
        if (j < 3) {
#pragma unroll
            for (int b = 0; b < EB; ++b) {
                qsum[b] = j == 0 ? acc[b] : qsum[b] + acc[b];
                acc[b] = f32x4{0.f, 0.f, 0.f, 0.f};
            }
        }
    }
#pragma unroll
    for (int b = 0; b < EB; ++b) acc[b] = qsum[b] + acc[b];  // + q3
    // ---- selection from the accumulators: round r routes token 4 kg + r of each DPP row ----
#pragma unroll
    for (int r = 0; r < 4; ++r) {
        float v[EB];
#pragma unroll
        for (int b = 0; b < EB; ++b) v[b] = acc[b][r];
        const int t = t0 + wave * 16 + 4 * kg + r;
        const bool active = t < T;
        const int tr = active ? t : 0;
        select_vals<EB>(v, E, K, active, expert_ids + static_cast<size_t>(tr) * K, weights + static_cast<size_t>(tr) * K);
    }
    // ---- optional tail: the block's slots ranked by expert, for the permute's scatter ----
    if (counts != nullptr) {
        __syncthreads();  // the block's ids are written and the stages are no longer read
        constexpr int MAXIT = (kRowTokens * kRankTopK + kRowWaves * kWave - 1) / (kRowWaves * kWave);
        rank_slots<kRowWaves, MAXIT>(expert_ids, t0 * K, min(T, t0 + kRowTokens) * K, E, counts_stride(E),
                                     reinterpret_cast<int*>(lds),
                                     counts + static_cast<size_t>(blockIdx.x) * counts_stride(E), rank);
    }
}

// ---- the quarters kernel: one 16-token block per workgroup, wave j sums quarter j of the stages ----
// With few tokens the rows kernel's 64-token workgroups leave most CUs idle and every wave multiplies all of
// w_gate. Here a workgroup owns 16 tokens and each of its 4 waves streams one quarter of the stages through
// double-buffered stages of its own (w_gate 16 KB, x SK KB), with no barrier in the loop: a wave reads only what
// its own copies wrote. The compiler waits for every direct-to-LDS copy in flight (vmcnt(0)) before a
// ds_read_b64_tr_b16 that follows it, since it cannot tell which LDS bytes a copy writes, so a stage is read
// whole into registers before the next stage's copies go out; those then land while the stage's MFMAs run.
// Wave 0 then adds the other waves' sums in quarter order, ((q0 + q1) + q2) + q3 as the rows kernel does, and
// selects.
constexpr size_t quarter_lds_bytes(int eb) { return 4 * (2 * size_t(16384) + 2 * size_t(row_stage_ksteps(eb)) * 1024); }

template <int EB>
__global__ __launch_bounds__(4 * kWave) void routing_quarters_kernel(const uint16_t* __restrict__ x,
                                                                     const uint16_t* __restrict__ w_gate,
                                                                     int32_t* __restrict__ expert_ids,
                                                                     uint16_t* __restrict__ weights, int T, int H,
                                                                     int E, int K, int32_t* __restrict__ counts,
                                                                     int32_t* __restrict__ rank) {
    constexpr int Epad = EB * 16;
    constexpr int SK = row_stage_ksteps(EB);
    constexpr int kStage = SK * 32 * Epad * 2;
    constexpr int kWaveLds = 2 * kStage + 2 * SK * 1024;
    static_assert(kStage == 16384, "stage geometry");
    extern __shared__ __align__(16) uint8_t lds[];
    const int lane = lane_id();
    const int wave = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x) / kWave);
    uint8_t* wbuf = lds + wave * kWaveLds;  // [2][kStage]
    uint8_t* xbuf = wbuf + 2 * kStage;       // [2][SK][16 rows][64 B]
    const int t0 = static_cast<int>(blockIdx.x) * 16;
    const int nst = H / 32 / SK;  // the host runs this kernel only when SK divides H / 32
    const int s0 = quarter_begin(wave, nst);
    const int n = quarter_begin(wave + 1, nst) - s0;  // this wave's stages: s0 .. s0 + n - 1

    const __amdgpu_buffer_rsrc_t wrs =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t*>(w_gate), 0, H * E * 2, 0x00020000);
    const __amdgpu_buffer_rsrc_t xrs = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<uint16_t*>(x + static_cast<size_t>(t0) * H), 0, min(16, T - t0) * H * 2, 0x00020000);
    // x copy: lane -> row lane / 4 (token t0 + row, clamped into the batch), 16-byte chunk lane % 4
    const int xoff = (min(lane / 4, T - 1 - t0) * H + (lane % 4) * 8) * 2;
    // w_gate copy: the wave fills all 16 slabs of 1 KB of its stage; lane -> 16-byte slot of the slab
    int woff[16];
#pragma unroll
    for (int m = 0; m < 16; ++m) {
        const int off = m * 1024 + lane * 16;
        const int R = off / (32 * EB), pc = (off % (32 * EB)) / 16;  // stage row (SK k-steps of 32), slot
        const int c = pc ^ ((R % 32) & (2 * EB - 1));                 // the logical chunk stored in slot pc
        woff[m] = (R * E + (c * 8 < E ? c * 8 : 0)) * 2;              // padding chunks copy any valid chunk
    }
    const int arow = lane & 15, kg = lane >> 4;
    int frag_off[2][EB];
    {
        const int sl = lane & 15;
#pragma unroll
        for (int h = 0; h < 2; ++h)
#pragma unroll
            for (int b = 0; b < EB; ++b) {
                const int r = 8 * kg + 4 * h + sl / 4;
                const int e = 16 * b + 4 * (sl % 4);
                frag_off[h][b] = wstage_chunk<EB>(r, e / 8) + (e % 8) * 2;
            }
    }
    auto issue = [&](int l) __attribute__((always_inline)) {  // this wave's stage s0 + l
        uint8_t* dst = wbuf + (l & 1) * kStage;
#pragma unroll
        for (int m = 0; m < 16; ++m)
            __builtin_amdgcn_raw_ptr_buffer_load_lds(wrs, (__attribute__((address_space(3))) void*)(dst + m * 1024), 16,
                                                     static_cast<int>(woff[m]), (s0 + l) * SK * 32 * E * 2, 0, 0);
#pragma unroll
        for (int ks = 0; ks < SK; ++ks)
            __builtin_amdgcn_raw_ptr_buffer_load_lds(xrs, (__attribute__((address_space(3))) void*)(xbuf + ((l & 1) * SK + ks) * 1024),
                                                     16, xoff, ((s0 + l) * SK + ks) * 64, 0, 0);
    };

    f32x4 acc[EB];
#pragma unroll
    for (int b = 0; b < EB; ++b) acc[b] = f32x4{0.f, 0.f, 0.f, 0.f};
    if (n > 0) issue(0);
    for (int l = 0; l < n; ++l) {
        __builtin_amdgcn_s_waitcnt(vmcnt_imm(0));  // this wave's copies of stage l (the only ones in flight)
        const uint8_t* ws = wbuf + (l & 1) * kStage;
        const uint8_t* xs = xbuf + (l & 1) * SK * 1024;
        f16x8 a[SK], bv[SK][EB];
#pragma unroll
        for (int ks = 0; ks < SK; ++ks) {
            a[ks] = *reinterpret_cast<const f16x8*>(xs + ks * 1024 + arow * 64 + kg * 16);
            const uint8_t* wk = ws + ks * 32 * Epad * 2;
#pragma unroll
            for (int b = 0; b < EB; ++b) {
                const s16x4 lo = lds_read_tr16(wk + frag_off[0][b]);
                const s16x4 hi = lds_read_tr16(wk + frag_off[1][b]);
                bv[ks][b] = __builtin_bit_cast(f16x8, __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7));
            }
        }
        // stage l + 1 refills the buffers of stage l - 1, whose reads fed MFMAs in the previous iteration
        if (l + 1 < n) issue(l + 1);
#pragma unroll
        for (int ks = 0; ks < SK; ++ks)
#pragma unroll
            for (int b = 0; b < EB; ++b) acc[b] = mfma16x16x32(a[ks], bv[ks][b], acc[b]);
    }
    // waves 1-3 park their quarter sums in their own (idle) w_gate buffers: lane-major f32x4 per expert block
    if (wave > 0) {
#pragma unroll
        for (int b = 0; b < EB; ++b) *reinterpret_cast<f32x4*>(wbuf + (b * kWave + lane) * 16) = acc[b];
    }
    __syncthreads();
    if (wave == 0) {
#pragma unroll
        for (int j = 1; j < 4; ++j)
#pragma unroll
            for (int b = 0; b < EB; ++b)
                acc[b] = acc[b] + *reinterpret_cast<const f32x4*>(lds + j * kWaveLds + (b * kWave + lane) * 16);
        // ---- selection from the sums: round r routes token 4 kg + r of each DPP row ----
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            float v[EB];
#pragma unroll
            for (int b = 0; b < EB; ++b) v[b] = acc[b][r];
            const int t = t0 + 4 * kg + r;
            const bool active = t < T;
            const int tr = active ? t : 0;
            select_vals<EB>(v, E, K, active, expert_ids + static_cast<size_t>(tr) * K,
                            weights + static_cast<size_t>(tr) * K);
        }
    }
    // ---- optional tail: the block's slots ranked by expert, for the permute's scatter ----
    if (counts != nullptr) {
        __syncthreads();  // the block's ids are written and the sums are no longer read
        constexpr int MAXIT = (16 * kRankTopK + 4 * kWave - 1) / (4 * kWave);
        rank_slots<4, MAXIT>(expert_ids, t0 * K, min(T, t0 + 16) * K, E, counts_stride(E), reinterpret_cast<int*>(lds),
                             counts + static_cast<size_t>(blockIdx.x) * counts_stride(E), rank);
    }
}

// ---- split routing of one 16-token block (moe_layer, E > 64, T <= 16) ----
// At T <= 16 the quarters kernel's one workgroup reads all of w_gate on one CU (3.7 MB at E = 256, H = 7168:
// ~50 us). Here workgroup (j, g) runs quarter j of the quarters kernel's k-steps for the kSplitGB expert blocks
// of group g only (one wave), and writes its fp32 sums to the layer's workspace; a second launch adds the
// quarters as the quarters kernel does, ((q0 + q1) + q2) + q3, and selects. Every expert's sum runs the same
// MFMAs on the same fragments in the same k order, so ids and weights are the quarters kernel's bit for bit; only
// the staging differs (a window of 16 kSplitGB experts, stages of kSplitSK k-steps).
constexpr int kSplitGB = 2;
constexpr int kSplitSK = row_stage_ksteps(kSplitGB);  // 8 k-steps of 32 rows x 32 experts: 16 KB per stage
constexpr size_t kSplitLds = 2 * (16384 + size_t(kSplitSK) * 1024);

template <int EB>
__global__ __launch_bounds__(kWave) void routing_split_partial_kernel(const uint16_t* __restrict__ x,
                                                                      const uint16_t* __restrict__ w_gate, int T,
                                                                      int H, int E, float* __restrict__ part) {
    constexpr int GB = kSplitGB, SK = kSplitSK;
    constexpr int Gpad = GB * 16;
    constexpr int kStage = SK * 32 * Gpad * 2;
    static_assert(kStage == 16384 && EB % GB == 0, "stage geometry");
    extern __shared__ __align__(16) uint8_t lds[];
    uint8_t* wbuf = lds;               // [2][kStage]
    uint8_t* xbuf = lds + 2 * kStage;  // [2][SK][16 rows][64 B]
    const int lane = lane_id();
    const int j = static_cast<int>(blockIdx.x) % 4, grp = static_cast<int>(blockIdx.x) / 4;
    const int e0 = grp * Gpad;  // first expert of the window
    // quarter j of the quarters kernel's k-steps (its stages hold row_stage_ksteps(EB) k-steps each); the host
    // runs this kernel only where SK divides every quarter
    constexpr int SKq = row_stage_ksteps(EB);
    const int nstq = H / 32 / SKq;
    const int k0 = SKq * quarter_begin(j, nstq);
    const int n = (SKq * quarter_begin(j + 1, nstq) - k0) / SK;
    const __amdgpu_buffer_rsrc_t wrs =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t*>(w_gate), 0, H * E * 2, 0x00020000);
    const __amdgpu_buffer_rsrc_t xrs = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t*>(x), 0, T * H * 2, 0x00020000);
    const int xoff = (min(lane / 4, T - 1) * H + (lane % 4) * 8) * 2;
    // w_gate copy: the quarters kernel's stage layout for GB blocks, columns e0 .. e0 + Gpad - 1 of each row
    int woff[16];
#pragma unroll
    for (int m = 0; m < 16; ++m) {
        const int off = m * 1024 + lane * 16;
        const int R = off / (32 * GB), pc = (off % (32 * GB)) / 16;
        const int c = pc ^ ((R % 32) & (2 * GB - 1));
        const int col = e0 + c * 8;
        woff[m] = (R * E + (col < E ? col : 0)) * 2;  // padding chunks copy any valid chunk
    }
    const int arow = lane & 15, kg = lane >> 4;
    int frag_off[2][GB];
    {
        const int sl = lane & 15;
#pragma unroll
        for (int h = 0; h < 2; ++h)
#pragma unroll
            for (int b = 0; b < GB; ++b) {
                const int r = 8 * kg + 4 * h + sl / 4;
                const int e = 16 * b + 4 * (sl % 4);
                frag_off[h][b] = wstage_chunk<GB>(r, e / 8) + (e % 8) * 2;
            }
    }
    auto issue = [&](int l) __attribute__((always_inline)) {
        uint8_t* dst = wbuf + (l & 1) * kStage;
#pragma unroll
        for (int m = 0; m < 16; ++m)
            __builtin_amdgcn_raw_ptr_buffer_load_lds(wrs, (__attribute__((address_space(3))) void*)(dst + m * 1024), 16,
                                                     static_cast<int>(woff[m]), (k0 + l * SK) * 32 * E * 2, 0, 0);
#pragma unroll
        for (int ks = 0; ks < SK; ++ks)
            __builtin_amdgcn_raw_ptr_buffer_load_lds(xrs, (__attribute__((address_space(3))) void*)(xbuf + ((l & 1) * SK + ks) * 1024),
                                                     16, xoff, (k0 + l * SK + ks) * 64, 0, 0);
    };
    f32x4 acc[GB];
#pragma unroll
    for (int b = 0; b < GB; ++b) acc[b] = f32x4{0.f, 0.f, 0.f, 0.f};
    if (n > 0) issue(0);
    for (int l = 0; l < n; ++l) {
        __builtin_amdgcn_s_waitcnt(vmcnt_imm(0));  // this wave's copies of stage l (the only ones in flight)
        const uint8_t* ws = wbuf + (l & 1) * kStage;
        const uint8_t* xs = xbuf + (l & 1) * SK * 1024;
        f16x8 a[SK], bv[SK][GB];
#pragma unroll
        for (int ks = 0; ks < SK; ++ks) {
            a[ks] = *reinterpret_cast<const f16x8*>(xs + ks * 1024 + arow * 64 + kg * 16);
            const uint8_t* wk = ws + ks * 32 * Gpad * 2;
#pragma unroll
            for (int b = 0; b < GB; ++b) {
                const s16x4 lo = lds_read_tr16(wk + frag_off[0][b]);
                const s16x4 hi = lds_read_tr16(wk + frag_off[1][b]);
                bv[ks][b] = __builtin_bit_cast(f16x8, __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7));
            }
        }
        if (l + 1 < n) issue(l + 1);  // refills the buffers of stage l - 1
#pragma unroll
        for (int ks = 0; ks < SK; ++ks)
#pragma unroll
            for (int b = 0; b < GB; ++b) acc[b] = mfma16x16x32(a[ks], bv[ks][b], acc[b]);
    }
#pragma unroll
    for (int b = 0; b < GB; ++b)
        *reinterpret_cast<f32x4*>(part + ((static_cast<size_t>(j) * EB + grp * GB + b) * kWave + lane) * 4) = acc[b];
}

// the quarters' sums in the quarters kernel's order, then its selection
template <int EB>
__global__ __launch_bounds__(kWave) void routing_split_select_kernel(const float* __restrict__ part,
                                                                     int32_t* __restrict__ expert_ids,
                                                                     uint16_t* __restrict__ weights, int T, int E,
                                                                     int K) {
    const int lane = lane_id(), kg = lane >> 4;
    f32x4 acc[EB];
#pragma unroll
    for (int b = 0; b < EB; ++b) acc[b] = *reinterpret_cast<const f32x4*>(part + (static_cast<size_t>(b) * kWave + lane) * 4);
#pragma unroll
    for (int j = 1; j < 4; ++j)
#pragma unroll
        for (int b = 0; b < EB; ++b)
            acc[b] = acc[b] + *reinterpret_cast<const f32x4*>(part + ((static_cast<size_t>(j) * EB + b) * kWave + lane) * 4);
#pragma unroll
    for (int r = 0; r < 4; ++r) {
        float v[EB];
#pragma unroll
        for (int b = 0; b < EB; ++b) v[b] = acc[b][r];
        const int t = 4 * kg + r;
        const bool active = t < T;
        const int tr = active ? t : 0;
        select_vals<EB>(v, E, K, active, expert_ids + static_cast<size_t>(tr) * K, weights + static_cast<size_t>(tr) * K);
    }
}

// ---- resident kernel: 32 < E <= 64 at large T, w_gate held in registers ----
// The narrow kernel's workgroups each route 16-64 tokens and multiply all of w_gate into them, so at T = 16384,
// E = 64 they read 128 MB of w_gate from L2 beside 64 MB of x, four dependent round trips a wave. This kernel is
// persistent (one workgroup per CU, a contiguous run of 16-token blocks each) and reads w_gate once per
// workgroup: its 8 waves hold every B fragment of the narrow kernel in VGPRs. x streams through an LDS ring of
// 32 KB slots (16 token rows x 1024 columns), copied straight from memory into LDS a few slots ahead.
// Same bits as the narrow kernel: its 4 waves are kept as virtual waves v (wave v's k-step pairs v, v + 4, ...,
// each pair's two k-steps in order, on the same MFMA chain), physical wave w runs virtual wave w / 2 for expert
// blocks 2 (w % 2) and 2 (w % 2) + 1, and the 4 partials are folded in virtual-wave order before the same
// selection. Fragments are read from the narrow kernel's w_gate stage layout (wstage_chunk, ds_read_b64_tr_b16).
// LDS of a ring slot: token row r at r * 2048 bytes; 16-byte granule g of the row at g ^ r, so the 16 rows an
// A-fragment read touches lie in distinct banks.
constexpr int kResWaves = 8;
constexpr int kResChunk = 1024;                                  // x columns per ring slot (32 k-steps)
constexpr int kResSlotBytes = 16 * kResChunk * 2;                // 32 KB
constexpr int kResCopies = kResSlotBytes / 1024 / kResWaves;     // 1 KB copies per wave and slot: 4
constexpr int kResEB = 4;                                        // expert blocks (32 < E <= 64)
constexpr int kResVW = waves_for(kResEB, 1);                     // the narrow kernel's waves: 4 virtual waves
constexpr int kResSlots = 4;                                     // ring slots
constexpr int kResSel = 4;  // token blocks whose folded logits wait for one selection round of all 8 waves
// ring, partials [4 virtual waves][16 tokens][64], logits [4 blocks][16 tokens][64]: 160 KB
constexpr size_t kResLdsBytes = static_cast<size_t>(kResSlots) * kResSlotBytes + (kResVW + kResSel) * 16 * 64 * 4;
// Workgroups of the persistent grid: one per CU of the MI355X.
constexpr int kResGrid = 256;
int res_blocks_per_wg(int T) {
    const int nblocks = (T + 15) / 16;
    return (nblocks + kResGrid - 1) / kResGrid;
}

// Barrier over this wave's LDS accesses only: the x copies in flight (vmcnt) are not waited for, as a
// workgroup-scope release fence would. The LDS writes before it are this wave's ds_writes (lgkmcnt) and the
// copies of slots the caller waited for explicitly.
__device__ __forceinline__ void lds_barrier_nowait() {
    __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0)
    __builtin_amdgcn_sched_barrier(0);
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
    __builtin_amdgcn_sched_barrier(0);
}

// Four ds_read_b64_tr_b16 and their wait as one inline-assembly statement. The compiler waits for every
// direct-to-LDS copy in flight before the builtin (it cannot tell which LDS bytes a copy writes), which would hold
// the fragment reads behind the x copies of the ring; here the registers are whole when the statement ends.
__device__ __forceinline__ uint32_t lds_addr(const uint8_t* p) {
    return static_cast<uint32_t>(reinterpret_cast<uintptr_t>((__attribute__((address_space(3))) const uint8_t*)(p)));
}
__device__ __forceinline__ void lds_read_tr16_x4(const uint8_t* p0, const uint8_t* p1, const uint8_t* p2,
                                                 const uint8_t* p3, s16x4 (&v)[4]) {
    asm volatile(
        "ds_read_b64_tr_b16 %0, %4\n\tds_read_b64_tr_b16 %1, %5\n\tds_read_b64_tr_b16 %2, %6\n\t"
        "ds_read_b64_tr_b16 %3, %7\n\ts_waitcnt lgkmcnt(0)"
        : "=&v"(v[0]), "=&v"(v[1]), "=&v"(v[2]), "=&v"(v[3])
        : "v"(lds_addr(p0)), "v"(lds_addr(p1)), "v"(lds_addr(p2)), "v"(lds_addr(p3)));
}

// NPV: k-step pairs per virtual wave (H = 256 NPV); a wave holds 4 NPV B fragments, 128 VGPRs at NPV = 8.
// x is loaded non-temporally: from 32768 tokens at H >= 1024 it is at least 64 MB (kNtXBytes).
template <int NPV>
__global__ __launch_bounds__(kResWaves * kWave) void routing_resident_kernel(const uint16_t* __restrict__ x,
                                                                             const uint16_t* __restrict__ w_gate,
                                                                             int32_t* __restrict__ expert_ids,
                                                                             uint16_t* __restrict__ weights, int T,
                                                                             int H, int E, int K, int bpw,
                                                                             int32_t* __restrict__ counts,
                                                                             int32_t* __restrict__ rank) {
    constexpr int EB = kResEB, VW = kResVW, R = kResSlots, SB = kResSel;
    constexpr int VPW = 1, BPW = 2;  // virtual waves and expert blocks of a physical wave
    constexpr int Epad = EB * 16;
    constexpr int PPC = 16 / VW;      // pairs of a virtual wave in one slot (32 k-steps = 16 pairs)
    constexpr int NCH = NPV / PPC;    // slots per token block: H / kResChunk
    static_assert(NCH * PPC == NPV && VPW * BPW * kResWaves == VW * EB, "resident geometry");
    extern __shared__ __align__(16) uint8_t lds[];
    float* part = reinterpret_cast<float*>(lds + R * kResSlotBytes);  // [VW][16 tokens][Epad]
    float* logit = part + VW * 16 * Epad;                              // [SB][16 tokens][Epad]
    const int lane = lane_id();
    const int wave = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x) / kWave);
    const int row = lane & 15, kg = lane >> 4;
    // this wave's virtual wave v0 and expert blocks b0, b0 + 1
    const int v0 = wave / (kResWaves / VW);
    const int b0 = (wave % (kResWaves / VW)) * BPW;
    const int nblocks = (T + 15) / 16;
    const int blk0 = static_cast<int>(blockIdx.x) * bpw;  // the host sizes the grid so that blk0 < nblocks
    const int blk1 = min(nblocks, blk0 + bpw);

    // ---- x ring: copy m of a wave fills 1 KB = half of token row r = 2 wave + m / 2 ----
    int xoff[kResCopies];
#pragma unroll
    for (int m = 0; m < kResCopies; ++m) {
        const int r = 2 * wave + m / 2;
        const int lg = (64 * (m & 1) + lane) ^ r;  // the logical granule stored in this lane's physical granule
        xoff[m] = r * H * 2 + lg * 16;
    }
    const int nq = (blk1 - blk0) * NCH;  // ring slots this workgroup runs through
    auto issue = [&](int qq) __attribute__((always_inline)) {
        const int b = blk0 + qq / NCH, c = qq % NCH;
        const __amdgpu_buffer_rsrc_t xrs = __builtin_amdgcn_make_buffer_rsrc(
            const_cast<uint16_t*>(x + static_cast<size_t>(b) * 16 * H), 0, min(16, T - b * 16) * H * 2, 0x00020000);
        uint8_t* dst = lds + (qq % R) * kResSlotBytes + wave * kResCopies * 1024;
#pragma unroll
        for (int m = 0; m < kResCopies; ++m)  // rows past T read zeros; their results are dropped
            __builtin_amdgcn_raw_ptr_buffer_load_lds(xrs, (__attribute__((address_space(3))) void*)(dst + m * 1024), 16,
                                                     xoff[m], c * kResChunk * 2, 0, 2 /* nt */);
    };
    const int nx0 = min(R - 1, nq);  // ring slots issued during the w_gate staging

    // ---- w_gate into registers: k-steps staged 32 rows at a time in the narrow kernel's layout, in the last ring
    // slot, the partials and the logits, while the x copies of the other slots are in flight ----
    f16x8 wf[VPW][BPW][NPV][2];
    {
        constexpr int kStep = EB * 1024;  // one k-step's 32 rows x Epad, 2 Epad 16-byte chunks a row
        constexpr int kStaging = static_cast<int>(kResLdsBytes) - (R - 1) * kResSlotBytes;
        uint8_t* stage0 = lds + (R - 1) * kResSlotBytes;
        const int kpp = kStaging / kStep;
        const int nsteps = H / 32;
        // copy j fills stage bytes [1024 j, 1024 j + 1024); a wave's copies are j = wave (mod 8), so all of them
        // are chunk i = wave % EB of their k-step
        const int slot = (wave % EB) * kWave + lane;
        const int r = slot / (2 * EB), pc = slot % (2 * EB);
        const int c = pc ^ (r & (2 * EB - 1));
        const int cpy = (r * E + (c * 8 < E ? c * 8 : 0)) * 2;  // padding chunks copy any valid chunk
        int frag_off[2][BPW];
        const int sl = lane & 15;
#pragma unroll
        for (int h = 0; h < 2; ++h)
#pragma unroll
            for (int bi = 0; bi < BPW; ++bi) {
                const int rr = 8 * kg + 4 * h + sl / 4;
                const int e = 16 * (b0 + bi) + 4 * (sl % 4);
                frag_off[h][bi] = wstage_chunk<EB>(rr, e / 8) + (e % 8) * 2;
            }
        const __amdgpu_buffer_rsrc_t wrs =
            __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t*>(w_gate), 0, H * E * 2, 0x00020000);
        for (int ks0 = 0; ks0 < nsteps; ks0 += kpp) {
            const int nks = min(kpp, nsteps - ks0);
            if (ks0 > 0) lds_barrier_nowait();  // every wave has read the previous pass's stages
            for (int j = wave; j < nks * EB; j += kResWaves)
                __builtin_amdgcn_raw_ptr_buffer_load_lds(wrs, (__attribute__((address_space(3))) void*)(stage0 + j * 1024), 16,
                                                         cpy, (ks0 + j / EB) * 32 * E * 2, 0, 0);
            if (ks0 == 0) {  // the x slots go out behind the first pass's copies, which are waited for alone
                for (int qq = 0; qq < nx0; ++qq) issue(qq);
                if (nx0 >= 3) __builtin_amdgcn_s_waitcnt(vmcnt_imm(3 * kResCopies));
                else if (nx0 == 2) __builtin_amdgcn_s_waitcnt(vmcnt_imm(2 * kResCopies));
                else __builtin_amdgcn_s_waitcnt(vmcnt_imm(kResCopies));
            } else {
                __builtin_amdgcn_s_waitcnt(vmcnt_imm(0));
            }
            lds_barrier_nowait();  // (a workgroup release fence would wait for the x copies as well)
#pragma unroll
            for (int vi = 0; vi < VPW; ++vi)
#pragma unroll
                for (int ii = 0; ii < NPV; ++ii)
#pragma unroll
                    for (int st = 0; st < 2; ++st) {
                        const int ks = 2 * (v0 + vi + ii * VW) + st;
                        if (ks < ks0 || ks >= ks0 + nks) continue;  // uniform
                        const uint8_t* stg = stage0 + (ks - ks0) * kStep;
                        s16x4 v[4];  // halves lo, hi of expert blocks b0, b0 + 1
                        lds_read_tr16_x4(stg + frag_off[0][0], stg + frag_off[1][0], stg + frag_off[0][1],
                                         stg + frag_off[1][1], v);
#pragma unroll
                        for (int bi = 0; bi < BPW; ++bi)
                            wf[vi][bi][ii][st] = __builtin_bit_cast(f16x8, __builtin_shufflevector(v[2 * bi], v[2 * bi + 1], 0, 1, 2, 3, 4, 5, 6, 7));
                    }
        }
        lds_barrier_nowait();  // every wave's fragments are in registers before the ring overwrites the stages
    }


    constexpr int G = narrow_sel_lanes(EB);
    constexpr int TPW = kWave / G;
    int q = 0;
    for (int b = blk0; b < blk1; ++b) {
        f32x4 acc[VPW][BPW];
#pragma unroll
        for (int vi = 0; vi < VPW; ++vi)
#pragma unroll
            for (int bi = 0; bi < BPW; ++bi) acc[vi][bi] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int c = 0; c < NCH; ++c, ++q) {
            // this wave's copies of slot q have landed (those of up to R - 2 later slots may be in flight) ...
            const int ahead = min(R - 2, nq - 1 - q);
            if (ahead >= 2) __builtin_amdgcn_s_waitcnt(vmcnt_imm(2 * kResCopies));
            else if (ahead == 1) __builtin_amdgcn_s_waitcnt(vmcnt_imm(kResCopies));
            else __builtin_amdgcn_s_waitcnt(vmcnt_imm(0));
            lds_barrier_nowait();  // its reads of slot q - 1 are done, and every wave's: slot q is whole, q - 1 free
            if (q + R - 1 < nq) issue(q + R - 1);
            const uint8_t* xs = lds + (q % R) * kResSlotBytes + row * 2048;
#pragma unroll
            for (int vi = 0; vi < VPW; ++vi)
#pragma unroll
                for (int ii = c * PPC; ii < (c + 1) * PPC; ++ii)
#pragma unroll
                    for (int st = 0; st < 2; ++st) {
                        const int ksl = 2 * (v0 + vi + ii * VW) + st - 32 * c;  // k-step within the slot
                        const f16x8 a = *reinterpret_cast<const f16x8*>(xs + (((ksl * 4 + kg) ^ row) << 4));
#pragma unroll
                        for (int bi = 0; bi < BPW; ++bi) acc[vi][bi] = mfma16x16x32(a, wf[vi][bi][ii][st], acc[vi][bi]);
                    }
        }
        // partial logits of each virtual wave: D[token 4 kg + r][expert 16 b + row]
#pragma unroll
        for (int vi = 0; vi < VPW; ++vi)
#pragma unroll
            for (int bi = 0; bi < BPW; ++bi)
#pragma unroll
                for (int r = 0; r < 4; ++r)
                    part[((v0 + vi) * 16 + kg * 4 + r) * Epad + (b0 + bi) * 16 + row] = acc[vi][bi][r];
        lds_barrier_nowait();
        // fold in virtual-wave order into the block's logits rows
        const int lb = (b - blk0) % SB;
        const f32x4* part4 = reinterpret_cast<const f32x4*>(part);
        f32x4* logit4 = reinterpret_cast<f32x4*>(logit + lb * 16 * Epad);
        for (int i = static_cast<int>(threadIdx.x); i < 16 * Epad / 4; i += kResWaves * kWave) {
            f32x4 v = part4[i];
#pragma unroll
            for (int w = 1; w < VW; ++w) v += part4[w * 16 * Epad / 4 + i];
            logit4[i] = v;
        }
        // selection of the blocks held, all waves at once: G lanes per token, TPW tokens a wave. The next block's
        // partials are written after a ring barrier, which every wave reaches after its fold reads.
        if (lb == SB - 1 || b == blk1 - 1) {
            lds_barrier_nowait();
            const int tb0 = (b - lb) * 16;  // the first token of the blocks held
            const int nt = (lb + 1) * 16;
            for (int tw = wave * TPW; tw < nt; tw += kResWaves * TPW) {  // uniform: every lane joins the DPP steps
                const int t = tw + lane / G;
                const bool active = t < nt && tb0 + t < T;
                const int tr = min(t, nt - 1);  // inactive groups read a valid row and write nothing
                select_row<Epad / G, G>(logit + tr * Epad, E, K, active, expert_ids + static_cast<size_t>(tb0 + tr) * K,
                                        weights + static_cast<size_t>(tb0 + tr) * K);
            }
        }
    }
    // ---- optional tail: the workgroup's slots ranked by expert, for the permute's scatter ----
    if (counts != nullptr) {
        __syncthreads();  // the workgroup's ids are written and part[] is no longer read
        rank_slots<kResWaves, 4>(expert_ids, blk0 * 16 * K, min(T, blk1 * 16) * K, E, counts_stride(E),
                                 reinterpret_cast<int*>(part), counts + static_cast<size_t>(blockIdx.x) * counts_stride(E),
                                 rank);
    }
}

size_t wide_lds_bytes(int eb) {
    const int pitch = eb == 8 ? wide_pitch(8) : wide_pitch(16);
    return static_cast<size_t>(2) * eb * 16 * pitch * sizeof(uint16_t) +
           static_cast<size_t>(kWideTokens) * eb * 16 * sizeof(float);
}

template <int EB>
hipError_t launch_wide(const uint16_t* x, const uint16_t* w_gate, int32_t* ids, uint16_t* w, int T, int H, int E,
                       int K, int32_t* counts, int32_t* rank, hipStream_t stream) {
    const int grid = (T + kWideTokens - 1) / kWideTokens;
    const size_t lds = wide_lds_bytes(EB);
    const hipError_t attr = ensure_lds_limit(reinterpret_cast<const void*>(&routing_wide_kernel<EB>),
                                             static_cast<int>(lds));
    if (attr != hipSuccess) return attr;
    TraceScope trace("moe_routing_topk", stream);
    routing_wide_kernel<EB><<<grid, kWideWaves * kWave, lds, stream>>>(x, w_gate, ids, w, T, H, E, K, counts, rank);
    return hipGetLastError();
}

template <int EB, int TB, bool LW, bool NTX>
hipError_t launch_narrow_nt(const uint16_t* x, const uint16_t* w_gate, int32_t* ids, uint16_t* w, int T, int H, int E,
                            int K, int32_t* counts, int32_t* rank, hipStream_t stream) {
    const int grid = (T + 16 * TB - 1) / (16 * TB);
    const size_t lds = narrow_lds_bytes(EB, TB, LW);
    const hipError_t attr = ensure_lds_limit(reinterpret_cast<const void*>(&routing_topk_kernel<EB, TB, LW, NTX>),
                                             static_cast<int>(lds));
    if (attr != hipSuccess) return attr;
    TraceScope trace("moe_routing_topk", stream);
    routing_topk_kernel<EB, TB, LW, NTX><<<grid, waves_for(EB, TB) * kWave, lds, stream>>>(x, w_gate, ids, w, T, H, E,
                                                                                         K, counts, rank);
    return hipGetLastError();
}

// x bytes from which the narrow kernel loads x non-temporally. In the layer, x has been partly evicted from the
// 256 MB Infinity Cache by the FFN's weights and intermediate when routing reads it again: at 64 MB (T = 16384,
// H = 2048, E = 64) the hint took routing from 26.7 to 24.7 us, at 32 MB (T = 8192, E = 16) it made it slower
// (11.5 against 11.0 us), and at decode (0.5 MB, cache-resident) it made the layer 2 us slower.
constexpr int64_t kNtXBytes = int64_t(48) << 20;

template <int EB, int TB, bool LW>
hipError_t launch_narrow(const uint16_t* x, const uint16_t* w_gate, int32_t* ids, uint16_t* w, int T, int H, int E,
                         int K, int32_t* counts, int32_t* rank, hipStream_t stream) {
    if constexpr (LW && TB >= 2) {
        if (static_cast<int64_t>(T) * H * 2 >= kNtXBytes)
            return launch_narrow_nt<EB, TB, LW, true>(x, w_gate, ids, w, T, H, E, K, counts, rank, stream);
    }
    return launch_narrow_nt<EB, TB, LW, false>(x, w_gate, ids, w, T, H, E, K, counts, rank, stream);
}

template <int EB, int TB>
hipError_t launch_narrow(const uint16_t* x, const uint16_t* w_gate, int32_t* ids, uint16_t* w, int T, int H, int E,
                         int K, int32_t* counts, int32_t* rank, hipStream_t stream) {
    return narrow_lds_weights(w_gate, H, E)
               ? launch_narrow<EB, TB, true>(x, w_gate, ids, w, T, H, E, K, counts, rank, stream)
               : launch_narrow<EB, TB, false>(x, w_gate, ids, w, T, H, E, K, counts, rank, stream);
}

template <int EB>
hipError_t launch_eb(const uint16_t* x, const uint16_t* w_gate, int32_t* ids, uint16_t* w, int T, int H, int E,
                     int K, int32_t* counts, int32_t* rank, hipStream_t stream) {
    switch (narrow_token_blocks(T, EB)) {
        case 1: return launch_narrow<EB, 1>(x, w_gate, ids, w, T, H, E, K, counts, rank, stream);
        case 2: return launch_narrow<EB, 2>(x, w_gate, ids, w, T, H, E, K, counts, rank, stream);
        default: return launch_narrow<EB, 4>(x, w_gate, ids, w, T, H, E, K, counts, rank, stream);
    }
}

template <int NPV>
hipError_t launch_resident(const uint16_t* x, const uint16_t* w_gate, int32_t* ids, uint16_t* w, int T, int H, int E,
                           int K, int32_t* counts, int32_t* rank, hipStream_t stream) {
    const int bpw = res_blocks_per_wg(T);
    const int grid = ((T + 15) / 16 + bpw - 1) / bpw;
    const hipError_t attr = ensure_lds_limit(reinterpret_cast<const void*>(&routing_resident_kernel<NPV>),
                                             static_cast<int>(kResLdsBytes));
    if (attr != hipSuccess) return attr;
    TraceScope trace("moe_routing_topk", stream);
    routing_resident_kernel<NPV><<<grid, kResWaves * kWave, kResLdsBytes, stream>>>(x, w_gate, ids, w, T, H, E, K, bpw,
                                                                                    counts, rank);
    return hipGetLastError();
}

// The resident kernel's shapes: 32 < E <= 64 (four expert blocks) and H = 1024 or 2048 (4 or 8 k-step pairs per
// virtual wave; whole 1024-column ring slots, the fragments within 128 VGPRs).
bool resident_shape(int H, int eb) { return eb == kResEB && (H == 1024 || H == 2048); }

template <int EB>
hipError_t launch_quarters(const uint16_t* x, const uint16_t* w_gate, int32_t* ids, uint16_t* w, int T, int H, int E,
                           int K, int32_t* counts, int32_t* rank, hipStream_t stream) {
    const int grid = (T + 15) / 16;
    const size_t lds = quarter_lds_bytes(EB);
    const hipError_t attr = ensure_lds_limit(reinterpret_cast<const void*>(&routing_quarters_kernel<EB>),
                                             static_cast<int>(lds));
    if (attr != hipSuccess) return attr;
    TraceScope trace("moe_routing_topk", stream);
    routing_quarters_kernel<EB><<<grid, 4 * kWave, lds, stream>>>(x, w_gate, ids, w, T, H, E, K, counts, rank);
    return hipGetLastError();
}

template <int EB>
hipError_t launch_rows(const uint16_t* x, const uint16_t* w_gate, int32_t* ids, uint16_t* w, int T, int H, int E,
                       int K, int32_t* counts, int32_t* rank, hipStream_t stream) {
    const int grid = (T + kRowTokens - 1) / kRowTokens;
    const size_t lds = row_lds_bytes(EB);
    const hipError_t attr = ensure_lds_limit(reinterpret_cast<const void*>(&routing_rows_kernel<EB>),
                                             static_cast<int>(lds));
    if (attr != hipSuccess) return attr;
    TraceScope trace("moe_routing_topk", stream);
    routing_rows_kernel<EB><<<grid, kRowWaves * kWave, lds, stream>>>(x, w_gate, ids, w, T, H, E, K, counts, rank);
    return hipGetLastError();
}

// Which kernel routes: the narrow kernel for E <= 64; for E > 64 the rows kernel when its copies can run (lw:
// w_gate rows can be copied 16 bytes at a time, and whole stages of k-steps), else the wide kernel. The choice
// does not depend on T, so a token's ids and weights do not depend on the batch it is routed in.
enum RoutingKernel { kNarrowKernel, kWideKernel, kRowsKernel, kQuartersKernel, kResidentKernel };
// Tokens up to which the quarters kernel runs instead of the rows kernel (same bits). The rows kernel takes about
// the same time from T = 128 to 16384 (one workgroup per CU at most, each streaming all of w_gate): 215.6, 75.8,
// 66.5 and 39.0 us at T = 16384 for the four shapes below. The quarters kernel (us):
//   E = 256, H = 7168, K = 8: T = 128 46.9, 8192 113.8, 12288 167.0, 16384 220.6
//   E = 256, H = 2048, K = 8: T = 4096 30.7, 8192 58.9, 12288 86.0, 16384 113.0
//   E = 128, H = 4096, K = 8: T = 8192 47.0, 12288 69.3, 16384 91.0
//   E = 128, H = 2048, K = 6: T = 8192 32.0, 12288 46.6, 16384 61.7
constexpr int64_t kQuartersMaxTokens = 8192;
// Tokens from which 32 < E <= 64 routes through the resident kernel (same bits as the narrow kernel). Isolated
// launches at H = 2048, E = 64, K = 6, x streamed from HBM (non-temporal) / evicted first, us:
//   T =  4096: narrow 12.2 / 14.9,  resident 13.6 / 17.8
//   T =  8192: narrow 14.1 / 17.9,  resident 15.5 / 20.8
//   T = 16384: narrow 22.5 / 24.9,  resident 20.8 / 25.7  (in the DeepSeek-V2-Lite layer 23.3 against 24.1-24.4)
//   T = 32768: narrow 39.3 / 41.4,  resident 32.6 / 37.7
// Each CU stages all of w_gate once (256 KB through LDS, ~3-4 us, partly behind the first x slots) and selects its
// tokens at the end, where the narrow kernel's two workgroups per CU hide one's selection behind the other's
// loads: the resident kernel gains only once a CU routes 128 tokens or more.
constexpr int64_t kResidentMinTokens = 32768;
static_assert(kResidentMinTokens * 1024 * 2 >= kNtXBytes, "the resident kernel always loads x non-temporally");
RoutingKernel routing_kernel(int T, int H, int E, bool lw) {
    const int eb = routing_expert_blocks(E);
    if (eb <= 4) return lw && T >= kResidentMinTokens && resident_shape(H, eb) ? kResidentKernel : kNarrowKernel;
    const bool rows_ok = lw && (H / 32) % row_stage_ksteps(eb) == 0;
    if (!rows_ok) return kWideKernel;
    return T <= kQuartersMaxTokens ? kQuartersKernel : kRowsKernel;
}

template <int EB>
hipError_t launch_split(const uint16_t* x, const uint16_t* w_gate, int32_t* ids, uint16_t* w, int T, int H, int E,
                        int K, float* part, hipStream_t stream) {
    const hipError_t attr = ensure_lds_limit(reinterpret_cast<const void*>(&routing_split_partial_kernel<EB>),
                                             static_cast<int>(kSplitLds));
    if (attr != hipSuccess) return attr;
    TraceScope trace("moe_routing_topk", stream);
    routing_split_partial_kernel<EB><<<4 * (EB / kSplitGB), kWave, kSplitLds, stream>>>(x, w_gate, T, H, E, part);
    routing_split_select_kernel<EB><<<1, kWave, 0, stream>>>(part, ids, w, T, E, K);
    return hipGetLastError();
}

}  // namespace

bool routing_split_applies(int T, int H, int E, bool lw) {
    if (T < 1 || T > 16 || routing_kernel(T, H, E, lw) != kQuartersKernel) return false;
    const int skq = row_stage_ksteps(routing_expert_blocks(E)), nst = H / 32 / skq;
    for (int j = 0; j < 4; ++j)
        if (skq * (quarter_begin(j + 1, nst) - quarter_begin(j, nst)) % kSplitSK != 0) return false;
    return true;
}

size_t routing_split_workspace_bytes(int T, int E) {
    return T <= 16 && E > 64 ? static_cast<size_t>(4) * 16 * kWave * 16 : 0;  // [4 quarters][16 blocks][64 lanes] f32x4
}

hipError_t launch_routing_split(const uint16_t* x, const uint16_t* w_gate, int32_t* ids, uint16_t* w, int T, int H,
                                int E, int K, float* part, hipStream_t stream) {
    return routing_expert_blocks(E) == 8 ? launch_split<8>(x, w_gate, ids, w, T, H, E, K, part, stream)
                                         : launch_split<16>(x, w_gate, ids, w, T, H, E, K, part, stream);
}

int routing_expert_blocks(int E) {
    const int eb = (E + 15) / 16;
    if (eb <= 1) return 1;
    if (eb <= 2) return 2;
    if (eb <= 4) return 4;
    if (eb <= 8) return 8;
    return 16;
}

bool routing_lds_weights(const void* w_gate, int H, int E) { return narrow_lds_weights(w_gate, H, E); }

int routing_tokens_per_block(int T, int H, int E, bool lw) {
    const int eb = routing_expert_blocks(E);
    switch (routing_kernel(T, H, E, lw)) {
        case kRowsKernel: return kRowTokens;
        case kQuartersKernel: return 16;
        case kResidentKernel: return 16 * res_blocks_per_wg(T);
        case kWideKernel: return kWideTokens;
        default: return kTokensPerBlock * narrow_token_blocks(T, eb);
    }
}
int routing_block_threads(int T, int H, int E, bool lw) {
    const int eb = routing_expert_blocks(E);
    switch (routing_kernel(T, H, E, lw)) {
        case kRowsKernel: return kRowWaves * kWave;
        case kQuartersKernel: return 4 * kWave;
        case kResidentKernel: return kResWaves * kWave;
        case kWideKernel: return kWideWaves * kWave;
        default: return waves_for(eb, narrow_token_blocks(T, eb)) * kWave;
    }
}
int routing_lds_bytes(int T, int H, int E, bool lw) {
    const int eb = routing_expert_blocks(E);
    switch (routing_kernel(T, H, E, lw)) {
        case kRowsKernel: return static_cast<int>(row_lds_bytes(eb));
        case kQuartersKernel: return static_cast<int>(quarter_lds_bytes(eb));
        case kResidentKernel: return static_cast<int>(kResLdsBytes);
        case kWideKernel: return static_cast<int>(wide_lds_bytes(eb));
        default: return static_cast<int>(narrow_lds_bytes(eb, narrow_token_blocks(T, eb), lw));
    }
}
int routing_blocks(int T, int H, int E, bool lw) {
    const int tpb = routing_tokens_per_block(T, H, E, lw);
    return (T + tpb - 1) / tpb;
}

hipError_t launch_routing_topk(const uint16_t* x, const uint16_t* w_gate, int32_t* ids, uint16_t* w, int T, int H,
                               int E, int K, hipStream_t stream, int32_t* counts, int32_t* rank) {
    const int eb = routing_expert_blocks(E);
    switch (routing_kernel(T, H, E, narrow_lds_weights(w_gate, H, E))) {
        case kRowsKernel:
            return eb == 8 ? launch_rows<8>(x, w_gate, ids, w, T, H, E, K, counts, rank, stream)
                           : launch_rows<16>(x, w_gate, ids, w, T, H, E, K, counts, rank, stream);
        case kQuartersKernel:
            return eb == 8 ? launch_quarters<8>(x, w_gate, ids, w, T, H, E, K, counts, rank, stream)
                           : launch_quarters<16>(x, w_gate, ids, w, T, H, E, K, counts, rank, stream);
        case kResidentKernel:
            return H == 1024 ? launch_resident<4>(x, w_gate, ids, w, T, H, E, K, counts, rank, stream)
                             : launch_resident<8>(x, w_gate, ids, w, T, H, E, K, counts, rank, stream);
        default: break;
    }
    switch (eb) {
        case 1: return launch_eb<1>(x, w_gate, ids, w, T, H, E, K, counts, rank, stream);
        case 2: return launch_eb<2>(x, w_gate, ids, w, T, H, E, K, counts, rank, stream);
        case 4: return launch_eb<4>(x, w_gate, ids, w, T, H, E, K, counts, rank, stream);
        case 8: return launch_wide<8>(x, w_gate, ids, w, T, H, E, K, counts, rank, stream);
        default: return launch_wide<16>(x, w_gate, ids, w, T, H, E, K, counts, rank, stream);
    }
}

}  // namespace moe
