// moe_ffn_tiled.hip -- LDS-tiled schedule of the MoeExpertFFN grouped GEMMs (many rows per expert, prefill).
//
// Reference: op_kernel/moe_expert_ffn.cpp (ComputeSwiGLU :265-333, ComputeDownProj :339-394, scatter :250-257);
// oracle: tests/moe_cpu_sim.cpp:245-296 (W_gate, W_up [I, H]; W_down [H, I]).
//
// With ~1000 rows per expert (T = 8192, K = 2, E = 16) the GEMMs have an arithmetic intensity of ~1500 flop/B
// against HBM, far above the MFMA ridge. Both are "NT": activation rows and weight rows are contiguous along the
// reduction dim k.
//   macro tile   256 activation rows x 256 weight rows x 64 k per stage; 8 waves (2 x 4), each a 128 x 64
//                sub-tile (8 x 4 v_mfma_f32_16x16x32_f16 tiles, 128 fp32 accumulators per lane). The weight
//                fragment is the MFMA's first operand, so each lane ends with 4 consecutive output columns of one
//                row and the epilogue stores 8 bytes at a time.
//   copies       each stage is copied from global memory straight into LDS (buffer_load ... lds: no staging
//                registers, no LDS store instructions; 32-bit offsets against buffer resources whose range ends
//                at the buffer, so a read past it returns zeros instead of faulting)
//   ring         two LDS slots. Stage q's 64 MFMAs per wave run in four phases of 16; the LDS fragment reads a
//                later phase needs are issued between the MFMAs of the phase before (sched_group_barrier), so
//                both pipes stay busy. One barrier per stage, between the third and the fourth phase: by then
//                the wave has read all of stage q, and stage q + 1 has landed, so the barrier publishes q + 1
//                and frees q's slot for the copies of q + 2.
//   persistent   one workgroup per CU walks its tiles back to back and the ring runs on across them: the
//                copies of a tile's first two stages go out during the previous tile's last two. The tile table
//                (per-expert tile prefix and row offsets) is built once per workgroup in LDS, so finding a tile
//                is a short LDS binary search; the next tile's 256 sorted-slot entries are copied into LDS a tile
//                ahead.
//   split        (down) the down projection has only ~2 tiles per CU at prefill, so a count-based schedule
//                leaves the last round mostly idle: the tiles left over after the full rounds are split over k
//                into pieces, one per workgroup, that write fp32 partial tiles; ffn_tiled_fixup_kernel adds them
//                in piece order. The split is a separate instantiation (SPLIT), so gate/up keeps its register
//                allocation at tile changes.
//   LDS layout   unpadded 128-byte rows of 8 granules of 16 B; granule g of row r is stored at g ^ ((r >> 1) & 7),
//                so the 16 rows one ds_read_b128 touches (same logical granule) spread over all banks
//   gate/up      the 256 weight rows of a tile are, per wave quarter, 32 W_gate rows and the matching 32 W_up
//                rows, so each wave holds gate and up of the same (row, i) and applies SwiGLU in registers
//                (hardware exp2 and reciprocal, ~1 ulp each), writing fp16 hidden rows
//   down         weight rows are W_down rows (output columns); the epilogue writes expert_out[slot] directly
//   scheduling   tiles are (expert, n-tile, m-tile) with m fastest. Workgroups are dispatched round-robin over
//                the 8 XCDs; each XCD owns a contiguous range of tiles, so the m-tiles that share a weight tile
//                share that XCD's L2.
// Rows past an expert's count are clamped to its last row on load and masked on store. A reduction extent that is
// an odd multiple of 32 ends with a half stage (KT instantiation): its upper 32 columns are cleared in LDS.

#include "moe_device.h"
#include "moe_launch.h"

namespace moe {

namespace {

constexpr int kBM = 256;           // activation rows per tile
constexpr int kBN = 256;           // weight rows per tile
constexpr int kBK = 64;            // k per stage
constexpr int kPitch = kBK;        // LDS row pitch in halfs (granules XOR-swizzled)
constexpr int kThreads = 512;      // 8 waves
constexpr int kStageHalfs = (kBM + kBN) * kPitch;
constexpr int kNStage = 2;
constexpr int kLdsBytes = kNStage * kStageHalfs * 2;  // the ring; the tile table follows it
constexpr int kEpiStageBytes = kThreads / kWave * 2048;  // down epilogue: 16 rows x 128 B per wave
// LDS of a launch: the ring, the tile table (tab, offs: 2 (E + 1) ints), three row tables, then (down) the
// epilogue's staging rows at the next 16-byte boundary
__host__ __device__ constexpr int tiled_epi_stage_offset(int E) { return (kLdsBytes + 8 * (E + 1) + 3 * kBM * 4 + 15) / 16 * 16; }
__host__ __device__ constexpr int tiled_lds_bytes(int E, bool down) {
    return down ? tiled_epi_stage_offset(E) + kEpiStageBytes : kLdsBytes + 8 * (E + 1) + 3 * kBM * 4;
}
constexpr int kLdsMax = 160 * 1024;
constexpr int kXcds = 8;
constexpr int kCopyPolicy = 1;  // cache-policy bits of the stage copies: sc0
// Partial tiles of the split leftover round: one fp32 kBM x kBN tile per workgroup of a persistent launch.
constexpr int kMaxParts = 256;
constexpr int kFixThreads = 256;
constexpr int kFixRows = 16;  // tile rows per fix-up workgroup
// The split pays off only while the leftover round is a large share of the down projection: at DeepSeek-V2-Lite
// prefill (T = 16384, E = 64, K = 6, 13-14 rounds of 22-stage tiles) the unsplit kernel takes 575 us against
// 589 us + a 15 us fix-up split; at 2-2.5 rounds (T = 8192, E = 16; Mixtral T = 4096) the split saves 100-215 us.
constexpr int kSplitMaxRounds = 4;

struct TiledArgs {
    const uint16_t* act;         // x [T, H] (gate/up, gathered) or hidden [T*K, I] (down)
    const int32_t* sorted_slot;
    const int32_t* offsets;
    const uint16_t* w;           // expert_weights
    uint16_t* out;               // hidden or expert_out
    int T, E, K, H, I;
    int kdim;                    // H or I
    int ndim;                    // I (gate/up: tile covers 128 i of gate and up) or H (down)
    int ntiles_n;                // n-tiles per expert
    int gather;                  // gate/up: activation row r -> x[sorted_slot[r] / K]
    int split;                   // split the leftover tiles of each XCD over k (persistent grid <= kMaxParts)
    float* partial;              // [kMaxParts, kBM, kBN] fp32 partial tiles of the split leftover round
};

// Work of one XCD: its tiles [base, base + n) are dealt to its nloc workgroups in R full rounds; the L tiles
// left over are each split over k into S pieces of at least two stages, one piece per workgroup, so the last
// round keeps every workgroup busy instead of L of them. S = 1 runs the leftover tiles whole.
struct XcdSched {
    int base, n, R, L, S;
};
__device__ __forceinline__ XcdSched xcd_sched(int x, int total, int nloc, int nst, int split) {
    XcdSched s;
    const int per_xcd = (total + kXcds - 1) / kXcds;
    s.base = x * per_xcd;
    s.n = max(0, min(per_xcd, total - s.base));
    s.R = s.n / nloc;
    s.L = s.n - s.R * nloc;
    s.S = 1;
    if (split && s.L > 0) s.S = max(1, min(nloc / s.L, nst / 2));
    return s;
}

// Barrier of the copy ring. The only LDS writes of the main loop are this wave's direct-to-LDS copies, which the
// caller's explicit vmcnt wait covers, and every fragment read of the stage has fed an MFMA before the wave gets
// here. A workgroup-scope release fence would also wait for the copies still in flight (vmcnt(0)).
__device__ __forceinline__ void ring_barrier() {
    __builtin_amdgcn_sched_barrier(0);
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
    __builtin_amdgcn_sched_barrier(0);
}

// silu(g) * u with the hardware exp2 and reciprocal (each about 1 ulp): g * rcp(1 + 2^(-g log2 e)) * u.
__device__ __forceinline__ float swiglu_fast(float g, float u) {
#pragma clang fp contract(off)
    const float e = __builtin_amdgcn_exp2f(g * -1.4426950408889634f);
    return g * __builtin_amdgcn_rcpf(1.0f + e) * u;
}

// The lane index read afresh. Values derived from lane_id() are loop-invariant, so the compiler computes them
// once and keeps them live across the main loop, where the accumulators and fragments leave no room for them:
// they are spilled, and each reload in the tile change or the epilogue waits (vmcnt) for every stage copy in
// flight. A volatile read cannot be hoisted, so what make_plan and the epilogue derive from it is recomputed there.
// Used by the down projection (spills 44 -> 28 and 24 -> 12 registers; on one box DeepSeek-V2-Lite down
// 606-608 -> 568-571 us, prefill 496-499 -> 488-491 us, Mixtral 874 -> 868-869 us). Gate/up keeps lane_id(): its
// code is unchanged, and with the fresh index it ran 0.5-1 % slower.
__device__ __forceinline__ int lane_fresh() {
    int v;
    asm volatile("v_mbcnt_lo_u32_b32 %0, -1, 0\n\tv_mbcnt_hi_u32_b32 %0, -1, %0" : "=v"(v));
    return v;
}

enum Epilogue { kSwiGLU = 0, kScatter = 1 };

// Interleave pattern of one 16-MFMA phase: NR LDS reads and NV global->LDS copies are issued one after each of
// its first MFMAs, so neither pipe waits for the other.
template <int NR, int NV>
__device__ __forceinline__ void phase_sched() {
#pragma unroll
    for (int q = 0; q < 16; ++q) {
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // MFMA
        if (q < NR) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);  // DS read
        if (q < NV) __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);  // VMEM read
    }
}

// One work item: tile (e, mt, nt), k-stages [k0, k0 + nk), and the partial slot it writes (-1: the whole k
// range, written through the epilogue).
struct TileRef {
    int e, mt, nt, off, ne;
    int k0, nk, part;
};

// Copy plan of one tile: per stage and operand, wave w issues 4 instructions j, each filling 8 whole LDS rows
// r = (4 w + j) * 8 + lane / 8 (128 B each); lane fetches global granule (lane % 8) ^ ((r >> 1) & 7). ao / bo
// are byte offsets of those granules at k = 0 in the activation and weight buffers ar / wr.
struct CopyPlan {
    uint32_t ao[4], bo[4];
    __amdgpu_buffer_rsrc_t ar, wr;
};

// SPLIT: the leftover round may be split over k (p.split); a separate instantiation, so the kernel without it
// keeps its register allocation at tile changes. KT: the reduction extent is an odd multiple of 32, so the last
// k-stage holds 32 valid columns; its copies read on into the next row (or past the buffer, as zeros), and the
// waves zero those granules in LDS before the stage is published.
template <int EPI, bool SPLIT, bool KT = false>
__global__ __launch_bounds__(kThreads) void ffn_tiled_kernel(TiledArgs p) {
    extern __shared__ __align__(16) uint16_t lds[];
    const int tid = static_cast<int>(threadIdx.x);
    const int wave = __builtin_amdgcn_readfirstlane(tid / kWave);
    const int lane = lane_id();
    const int row16 = lane & 15, kg = lane >> 4;
    const int wm = wave >> 2, wn = wave & 3;  // 2 x 4 waves: rows wm*128.., weight rows wn*64..

    // Tile table in LDS after the ring: tab[e] = tiles of the experts before e (tab[E] = all tiles), offs[e] =
    // first sorted row of expert e. Tiles are (expert, n-tile, m-tile), m fastest.
    int* tab = reinterpret_cast<int*>(lds + kNStage * kStageHalfs);
    int* offs = tab + (p.E + 1);
    // Three row tables of 256 sorted-slot entries, one per tile in flight (tile k uses table k % 3): the copy rows
    // of gate/up gather x rows by them, the down epilogue scatters by them. Wave 0 copies tile k + 1's table
    // straight into LDS at the start of tile k; it lands before the next ring barrier.
    int* rowtab = reinterpret_cast<int*>(lds + kNStage * kStageHalfs) + 2 * (p.E + 1);
    if (wave == 0) {
        int carry = 0;
        for (int base = 0; base <= p.E; base += kWave) {
            const int e = base + lane;
            int o0 = 0, tiles = 0;
            if (e <= p.E) {
                o0 = p.offsets[e];
                offs[e] = o0;
            }
            if (e < p.E) tiles = (p.offsets[e + 1] - o0 + kBM - 1) / kBM * p.ntiles_n;
            int incl = tiles;  // inclusive scan over the wave
#pragma unroll
            for (int d = 1; d < kWave; d <<= 1) {
                const int v = __shfl_up(incl, d, kWave);
                if (lane >= d) incl += v;
            }
            if (e < p.E) tab[e + 1] = carry + incl;
            carry += __shfl(incl, kWave - 1, kWave);
        }
        if (lane == 0) tab[0] = 0;
    }
    __syncthreads();
    const int total = tab[p.E];

    // Persistent: the grid is a multiple of 8 workgroups, at most one per CU. Workgroups are dispatched
    // round-robin over the 8 XCDs, so workgroup b runs on XCD x = b % 8 as that XCD's li = b / 8-th workgroup.
    // XCD x owns tiles [x * per_xcd, (x + 1) * per_xcd) (m-tiles of one weight tile are consecutive, so they
    // share that XCD's L2), and its workgroups take them round-robin: li, li + nloc, li + 2 nloc, ...; with
    // p.split the tiles left over after the full rounds are split over k (xcd_sched).
    const int nst = (p.kdim + kBK - 1) / kBK;  // >= 2
    const int nloc = static_cast<int>(gridDim.x) / kXcds;
    const int x = static_cast<int>(blockIdx.x) % kXcds, li = static_cast<int>(blockIdx.x) / kXcds;
    const int per_xcd = (total + kXcds - 1) / kXcds;
    XcdSched xs{};
    if (SPLIT) xs = xcd_sched(x, total, nloc, nst, p.split);
    auto tile_at = [&](int k, TileRef& T) __attribute__((always_inline)) -> bool {
        int t;
        T.k0 = 0;
        T.nk = nst;
        T.part = -1;
        if (!SPLIT) {
            const int loc = li + k * nloc;
            t = x * per_xcd + loc;
            if (loc >= per_xcd || t >= total) return false;
        } else {
            int loc;
            if (k < xs.R) {
                loc = li + k * nloc;
            } else if (k == xs.R && xs.S == 1) {
                if (li >= xs.L) return false;
                loc = xs.R * nloc + li;
            } else if (k == xs.R) {  // piece pc of leftover tile j
                const int j = li / xs.S, pc = li - j * xs.S;
                if (j >= xs.L) return false;
                loc = xs.R * nloc + j;
                T.k0 = pc * nst / xs.S;
                T.nk = (pc + 1) * nst / xs.S - T.k0;
                T.part = static_cast<int>(blockIdx.x);
            } else {
                return false;
            }
            t = xs.base + loc;
        }
        int lo = 0, hi = p.E;  // tab[lo] <= t < tab[hi]
        while (hi - lo > 1) {
            const int mid = (lo + hi) >> 1;
            if (__builtin_amdgcn_readfirstlane(tab[mid]) <= t) lo = mid;
            else hi = mid;
        }
        T.e = lo;
        T.off = __builtin_amdgcn_readfirstlane(offs[lo]);
        T.ne = __builtin_amdgcn_readfirstlane(offs[lo + 1]) - T.off;
        const int mtiles = (T.ne + kBM - 1) / kBM;
        const int local = t - __builtin_amdgcn_readfirstlane(tab[lo]);
        T.nt = local / mtiles;
        T.mt = local - T.nt * mtiles;
        return true;
    };
    TileRef cur;
    if (!tile_at(0, cur)) return;

    // activation rows a tile copies: gate/up gathers token rows (x), down reads its own sorted hidden rows
    const uint32_t act_rows = static_cast<uint32_t>(p.T);
    const uint32_t kbytes = static_cast<uint32_t>(p.kdim) * 2;
    const __amdgpu_buffer_rsrc_t srsrc = __builtin_amdgcn_make_buffer_rsrc(const_cast<int32_t*>(p.sorted_slot), 0,
                                                                          p.T * p.K * 4, 0x00020000);
    auto load_rows = [&](const TileRef& T, int buf) __attribute__((always_inline)) {
        if (wave == 0) {
#pragma unroll
            for (int jj = 0; jj < kBM / kWave; ++jj) {
                const int r = jj * kWave + lane;
                const int row = T.off + min(T.mt * kBM + r, T.ne - 1);
                __builtin_amdgcn_raw_ptr_buffer_load_lds(srsrc, (__attribute__((address_space(3))) void*)(rowtab + buf * kBM + jj * kWave), 4,
                                                         row * 4, 0, 0, 0);
            }
        }
    };
    auto make_plan = [&](const TileRef& T, int buf, CopyPlan& P) __attribute__((always_inline)) {
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            // the down projection reads the lane index afresh (lane_fresh)
            const int r = (wave * 4 + j) * 8 + ((EPI == kScatter ? lane_fresh() : lane) / 8);
            const uint32_t gq = static_cast<uint32_t>(((EPI == kScatter ? lane_fresh() : lane) % 8) ^ ((r >> 1) & 7));
            if (p.gather) {
                P.ao[j] = static_cast<uint32_t>(rowtab[buf * kBM + r] / p.K) * kbytes + gq * 16;
            } else {  // rows relative to the tile's first row
                P.ao[j] = static_cast<uint32_t>(min(r, T.ne - 1 - T.mt * kBM)) * kbytes + gq * 16;
            }
            if (EPI == kSwiGLU) {
                const int quarter = r >> 6, sub = r & 63;
                const int ic = min(T.nt * 128 + quarter * 32 + (sub & 31), p.I - 1);
                P.bo[j] = ((sub < 32 ? 0u : static_cast<uint32_t>(p.I)) + static_cast<uint32_t>(ic)) * static_cast<uint32_t>(p.H) * 2 + gq * 16;
            } else {
                const int n = min(T.nt * kBN + r, p.H - 1);
                P.bo[j] = (2u * static_cast<uint32_t>(p.I) * p.H + static_cast<uint32_t>(n) * p.I) * 2 + gq * 16;
            }
        }
        if (p.gather) {
            P.ar = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t*>(p.act), 0, static_cast<int>(act_rows * kbytes), 0x00020000);
        } else {  // the tile's own rows only: any T*K*I stays within 32-bit offsets
            const int row0 = T.off + T.mt * kBM;
            const int rows = min(kBM, T.ne - T.mt * kBM);
            P.ar = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t*>(p.act + static_cast<size_t>(row0) * p.kdim), 0,
                                                     static_cast<int>(static_cast<uint32_t>(rows) * kbytes), 0x00020000);
        }
        const size_t ebase = static_cast<size_t>(T.e) * 3 * static_cast<size_t>(p.I) * p.H;
        P.wr = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t*>(p.w + ebase), 0,
                                                 static_cast<int>(3u * static_cast<uint32_t>(p.I) * p.H * 2), 0x00020000);
    };

    // copies stage kc of plan P into ring slot q % 2. The data is consumed from LDS, so the loads bypass the L1
    // (sc0); they still allocate in L2, where the other m-tiles of the weight tile find them (a non-temporal hint
    // there made the kernel 35 % slower).
    auto copy = [&](int q, int kc, const CopyPlan& P) __attribute__((always_inline)) {
        const int kb = kc * kBK * 2;  // byte offset of the stage along k (scalar)
        uint16_t* sa = lds + (q % kNStage) * kStageHalfs;
        uint16_t* sb = sa + kBM * kPitch;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            __builtin_amdgcn_raw_ptr_buffer_load_lds(P.ar, (__attribute__((address_space(3))) void*)(sa + (wave * 4 + j) * 8 * kPitch), 16,
                                                     static_cast<int>(P.ao[j]), kb, 0, kCopyPolicy);
            __builtin_amdgcn_raw_ptr_buffer_load_lds(P.wr, (__attribute__((address_space(3))) void*)(sb + (wave * 4 + j) * 8 * kPitch), 16,
                                                     static_cast<int>(P.bo[j]), kb, 0, kCopyPolicy);
        }
    };
    f32x4 acc[8][4];
    // Fragment registers: the wave's 128 rows are two halves of 4 16-row blocks (A0, A1); the 64 weight rows are
    // 4 blocks, held for the even (Bx) and the odd (By) 32-k step of a stage.
    f16x8 A0[4], A1[4], Bx[4], By[4];
    const int sw = (row16 >> 1) & 7;
    auto rdA = [&](int q, int kk, int h, f16x8 (&a)[4]) __attribute__((always_inline)) {
        const uint16_t* sa = lds + (q % kNStage) * kStageHalfs + (wm * 128 + h * 64 + row16) * kPitch + (((kk * 4 + kg) ^ sw) * 8);
#pragma unroll
        for (int i = 0; i < 4; ++i) a[i] = *reinterpret_cast<const f16x8*>(sa + i * 16 * kPitch);
    };
    auto rdB = [&](int q, int kk, f16x8 (&bb)[4]) __attribute__((always_inline)) {
        const uint16_t* sb = lds + (q % kNStage) * kStageHalfs + (kBM + wn * 64 + row16) * kPitch + (((kk * 4 + kg) ^ sw) * 8);
#pragma unroll
        for (int j = 0; j < 4; ++j) bb[j] = *reinterpret_cast<const f16x8*>(sb + j * 16 * kPitch);
    };
    // D[weight row][activation row]: each lane ends with 4 consecutive output columns of one row
    auto mma = [&](int h, const f16x8 (&a)[4], const f16x8 (&bb)[4], bool zero) __attribute__((always_inline)) {
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int j = 0; j < 4; ++j)
                acc[h * 4 + i][j] = mfma16x16x32(bb[j], a[i], zero ? f32x4{0.f, 0.f, 0.f, 0.f} : acc[h * 4 + i][j]);
    };

    // The ring of two LDS slots runs over this workgroup's tiles back to back: ring index q counts stages over
    // all its tiles, and the copies of a tile's first two stages are issued during the previous tile's last two.
    // Stage q multiplies its two 32-k steps in four phases of 16 MFMAs: (kk0, A0), (kk0, A1), (kk1, A0),
    // (kk1, A1). Each phase reads the fragments that the next phase or the one after needs. Between the third and
    // the fourth phase the wave has read all of stage q from LDS: one barrier then publishes stage q + 1 (every
    // wave's copies have landed) and frees slot q % 2 for the copies of ring stage q + 2 (stage kc of plan P).
    // After the last tile those copies repeat its last stage into the free slot and the fourth phase reads
    // fragments nobody uses.
    // KT: this wave's copy rows of ring stage qn, logical granules 4-7 (k 32-63 of the stage) set to zero; the lane
    // that copied a granule clears it, after its own copies have landed (vmcnt) and before the barrier that
    // publishes the stage (the caller's lgkmcnt(0) covers these writes)
    auto zero_tail = [&](int qn) __attribute__((always_inline)) {
        uint16_t* sa = lds + (qn % kNStage) * kStageHalfs;
        uint16_t* sb = sa + kBM * kPitch;
        const int ln = lane_fresh();
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int r = (wave * 4 + j) * 8 + ln / 8;
            if (((ln % 8) ^ ((r >> 1) & 7)) >= 4) {
                *reinterpret_cast<u32x4*>(sa + (wave * 4 + j) * 8 * kPitch + ln * 8) = u32x4{0u, 0u, 0u, 0u};
                *reinterpret_cast<u32x4*>(sb + (wave * 4 + j) * 8 * kPitch + ln * 8) = u32x4{0u, 0u, 0u, 0u};
            }
        }
    };
    auto stage = [&](int q, bool first, int kc, const CopyPlan& P, bool tail_next) __attribute__((always_inline)) {
        __builtin_amdgcn_sched_barrier(0);
        mma(0, A0, Bx, first);
        rdA(q, 0, 1, A1);
        rdB(q, 1, By);
        phase_sched<8, 0>();
        __builtin_amdgcn_sched_barrier(0);
        mma(1, A1, Bx, first);
        rdA(q, 1, 0, A0);
        phase_sched<4, 0>();
        __builtin_amdgcn_sched_barrier(0);
        mma(0, A0, By, false);
        rdA(q, 1, 1, A1);
        phase_sched<4, 0>();
        __builtin_amdgcn_sched_barrier(0);
        __builtin_amdgcn_s_waitcnt(vmcnt_imm(0));  // this wave's copies of ring stage q + 1
        if (KT && tail_next) zero_tail(q + 1);
        __builtin_amdgcn_s_waitcnt(0xc07f);        // lgkmcnt(0): this wave's reads of ring stage q are done
        ring_barrier();
        copy(q + 2, kc, P);
        mma(1, A1, By, false);
        rdB(q + 1, 0, Bx);
        rdA(q + 1, 0, 0, A0);
        phase_sched<8, 8>();
        __builtin_amdgcn_sched_barrier(0);
    };

    // Down projection: the same stage as a ring of 4 activation blocks of 16 rows, each read 3 blocks ahead of its
    // MFMAs (16 blocks per stage, 8 per 32-k step, numbered on across stages so that block n sits in Ar[n % 4]),
    // and the 4 weight blocks of each step (B0 even, B1 odd). 48 fragment registers instead of 64: the split
    // kernel spills 24 registers instead of 57, and the down projection runs 0.5-3 % faster (prefill 508.6 ->
    // 498-499 us, DeepSeek-V2-Lite 627 -> 607 us, Mixtral 892 -> 888 us; gate/up ran 1 % slower this way). The
    // barrier comes before the odd step's seventh block, when the wave has read all of stage q; the last two
    // blocks read stage q + 1's B0 and first 3 blocks.
    f16x8 B0[4], B1[4], Ar[4];
    auto rdA1 = [&](int q, int kk, int i) __attribute__((always_inline)) -> f16x8 {
        return *reinterpret_cast<const f16x8*>(lds + (q % kNStage) * kStageHalfs + (wm * 128 + i * 16 + row16) * kPitch +
                                               (((kk * 4 + kg) ^ sw) * 8));
    };
    auto rdB1 = [&](int q, int kk, int j) __attribute__((always_inline)) -> f16x8 {
        return *reinterpret_cast<const f16x8*>(lds + (q % kNStage) * kStageHalfs + (kBM + wn * 64 + j * 16 + row16) * kPitch +
                                               (((kk * 4 + kg) ^ sw) * 8));
    };
    auto stage_ring = [&](int q, bool first, int kc, const CopyPlan& P, bool tail_next) __attribute__((always_inline)) {
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            __builtin_amdgcn_sched_barrier(0);
            Ar[(i + 3) % 4] = rdA1(q, (i + 3) / 8, (i + 3) % 8);
            if (i < 4) B1[i] = rdB1(q, 1, i);
#pragma unroll
            for (int j = 0; j < 4; ++j) acc[i][j] = mfma16x16x32(B0[j], Ar[i % 4], first ? f32x4{0.f, 0.f, 0.f, 0.f} : acc[i][j]);
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // MFMA
                if (u < (i < 4 ? 2 : 1)) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);  // DS read
            }
        }
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            __builtin_amdgcn_sched_barrier(0);
            if (i < 5) Ar[(i + 3) % 4] = rdA1(q, 1, i + 3);
            if (i == 6) {
                __builtin_amdgcn_s_waitcnt(vmcnt_imm(0));  // this wave's copies of ring stage q + 1
                if (KT && tail_next) zero_tail(q + 1);
                __builtin_amdgcn_s_waitcnt(0xc07f);        // lgkmcnt(0): this wave's reads of ring stage q are done
                ring_barrier();
                copy(q + 2, kc, P);
#pragma unroll
                for (int j = 0; j < 4; ++j) B0[j] = rdB1(q + 1, 0, j);
                Ar[0] = rdA1(q + 1, 0, 0);
                Ar[1] = rdA1(q + 1, 0, 1);
            }
            if (i == 7) Ar[2] = rdA1(q + 1, 0, 2);
#pragma unroll
            for (int j = 0; j < 4; ++j) acc[i][j] = mfma16x16x32(B1[j], Ar[(i + 8) % 4], acc[i][j]);
            if (i == 6) {
#pragma unroll
                for (int u = 0; u < 4; ++u) {
                    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // MFMA
                    __builtin_amdgcn_sched_group_barrier(0x020, 2, 0);  // 2 copies
                    if (u < 3) __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);  // 2 DS reads
                }
            } else {
#pragma unroll
                for (int u = 0; u < 4; ++u) {
                    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // MFMA
                    if (u == 0 && (i < 5 || i == 7)) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);  // DS read
                }
            }
        }
        __builtin_amdgcn_sched_barrier(0);
    };
    // tail_next: ring stage q + 1 is the last k-stage (KT)
    auto run_stage = [&](int q, bool first, int kc, const CopyPlan& P, bool tail_next) __attribute__((always_inline)) {
        if constexpr (EPI == kScatter) stage_ring(q, first, kc, P, tail_next);
        else stage(q, first, kc, P, tail_next);
    };

    CopyPlan plan;
    load_rows(cur, 0);
    __builtin_amdgcn_s_waitcnt(vmcnt_imm(0));
    __syncthreads();
    make_plan(cur, 0, plan);
    copy(0, SPLIT ? cur.k0 : 0, plan);
    __builtin_amdgcn_s_waitcnt(vmcnt_imm(0));  // this wave's copies of stage 0 are in LDS
    ring_barrier();                            // and every wave's
    copy(1, SPLIT ? cur.k0 + 1 : 1, plan);
    if constexpr (EPI == kScatter) {
#pragma unroll
        for (int j = 0; j < 4; ++j) B0[j] = rdB1(0, 0, j);
#pragma unroll
        for (int i = 0; i < 3; ++i) Ar[i] = rdA1(0, 0, i);
    } else {
        rdB(0, 0, Bx);
        rdA(0, 0, 0, A0);
    }
    int q0 = 0;  // ring index of the current item's first stage
    for (int k = 0;; ++k) {
        TileRef nxt;
        const bool has_next = tile_at(k + 1, nxt);
        // table k + 1 % 3 was last read two tiles ago; the barriers of tile k - 1 separate those reads from this copy
        if (has_next) load_rows(nxt, (k + 1) % 3);
        // the last two stages copy the next item's first two (or, after the last item, repeat this one's last)
        const int k0 = SPLIT ? cur.k0 : 0, nk = SPLIT ? cur.nk : nst;  // nk >= 2
        const int nk0 = SPLIT ? nxt.k0 : 0;
        const int kc0 = has_next ? nk0 : k0 + nk - 1, kc1 = has_next ? nk0 + 1 : k0 + nk - 1;
        const bool tail = KT && k0 + nk == nst;  // this item ends with the 32-column k-stage
        if (nk > 2) {
            run_stage(q0, true, k0 + 2, plan, false);
            for (int s = 1; s + 2 < nk; ++s) run_stage(q0 + s, false, k0 + s + 2, plan, false);
            if (has_next) make_plan(nxt, (k + 1) % 3, plan);
            run_stage(q0 + nk - 2, false, kc0, plan, tail);
            run_stage(q0 + nk - 1, false, kc1, plan, false);
        } else {  // the next tile's plan is needed before the first barrier: wait for its row table here
            __builtin_amdgcn_s_waitcnt(vmcnt_imm(0));
            __syncthreads();
            if (has_next) make_plan(nxt, (k + 1) % 3, plan);
            run_stage(q0, true, kc0, plan, tail);
            run_stage(q0 + 1, false, kc1, plan, false);
        }

        // ---- epilogue: acc[i][j] lane holds D[weight row 4*kg + r of block j][activation row row16 of block i],
        // i.e. 4 consecutive output columns of one row: one 8-byte store per (i, j) ----
        const int m = cur.mt * kBM + wm * 128 + row16;
        if (SPLIT && cur.part >= 0) {
            // a piece of a split tile: the raw fp32 sums of its k-range, [activation row][weight row] of the tile
            const int lane_e = lane_fresh(), row16 = lane_e & 15, kg = lane_e >> 4;
            float* dst = p.partial + static_cast<size_t>(cur.part) * (kBM * kBN) + (wm * 128 + row16) * kBN + wn * 64 + kg * 4;
#pragma unroll
            for (int i = 0; i < 8; ++i)
#pragma unroll
                for (int j = 0; j < 4; ++j) *reinterpret_cast<f32x4*>(dst + i * 16 * kBN + j * 16) = acc[i][j];
        } else if (EPI == kSwiGLU) {
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                if (m + i * 16 >= cur.ne) continue;
                uint16_t* dst = p.out + static_cast<size_t>(cur.off + m + i * 16) * p.I;
#pragma unroll
                for (int j = 0; j < 2; ++j) {
                    const int col = cur.nt * 128 + wn * 32 + j * 16 + kg * 4;
                    if (col >= p.I) continue;
                    const uint32_t lo = f32_to_f16_bits(swiglu_fast(acc[i][j][0], acc[i][j + 2][0])) |
                                        (static_cast<uint32_t>(f32_to_f16_bits(swiglu_fast(acc[i][j][1], acc[i][j + 2][1]))) << 16);
                    const uint32_t hi = f32_to_f16_bits(swiglu_fast(acc[i][j][2], acc[i][j + 2][2])) |
                                        (static_cast<uint32_t>(f32_to_f16_bits(swiglu_fast(acc[i][j][3], acc[i][j + 2][3]))) << 16);
                    *reinterpret_cast<uint2*>(dst + col) = make_uint2(lo, hi);
                }
            }
        } else {
            // Whole-line stores: the wave's 128 x 64 sub-tile leaves as 16 instructions of 8 rows x 128 B. Row
            // block i passes through the wave's own 2 KB of LDS (16 rows x 128 B; 16-byte granule g of row r at
            // g ^ (r & 7)): lane (row16, kg) writes its four packed 4-column groups, then lane L reads granule
            // L % 8 of row h * 8 + L / 8 (h = 0, 1). Stored straight from the MFMA layout (16 rows x 32 B per
            // instruction) the epilogue cost ~100 us per DeepSeek-V2-Lite down launch (T = 16384, E = 64, K = 6).
            uint8_t* stg = reinterpret_cast<uint8_t*>(lds) + tiled_epi_stage_offset(p.E) + wave * 2048;
            const int lane_e = lane_fresh(), row16 = lane_e & 15, kg = lane_e >> 4;
            const int rr = lane_e >> 3, gq = lane_e & 7;
            const int col = cur.nt * kBN + wn * 64 + gq * 8;
#pragma unroll
            for (int i = 0; i < 8; ++i) {
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const uint32_t lo = f32_to_f16_bits(acc[i][j][0]) | (static_cast<uint32_t>(f32_to_f16_bits(acc[i][j][1])) << 16);
                    const uint32_t hi = f32_to_f16_bits(acc[i][j][2]) | (static_cast<uint32_t>(f32_to_f16_bits(acc[i][j][3])) << 16);
                    *reinterpret_cast<uint2*>(stg + row16 * 128 + (((2 * j + (kg >> 1)) ^ (row16 & 7)) << 4) + ((kg & 1) << 3)) =
                        make_uint2(lo, hi);
                }
                // the reads take what other lanes of this wave just wrote (LDS operations of one wave run in order)
                __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
                __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
                u32x4 v[2];
#pragma unroll
                for (int h = 0; h < 2; ++h) v[h] = *reinterpret_cast<const u32x4*>(stg + (h * 8 + rr) * 128 + ((gq ^ rr) << 4));
                __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");  // read before the next block's writes
                __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
#pragma unroll
                for (int h = 0; h < 2; ++h) {
                    const int r = wm * 128 + i * 16 + h * 8 + rr;  // row of the tile
                    if (cur.mt * kBM + r >= cur.ne || col >= p.H) continue;
                    *reinterpret_cast<u32x4*>(p.out + static_cast<size_t>(rowtab[(k % 3) * kBM + r]) * p.H + col) = v[h];
                }
            }
        }
        if (!has_next) break;
        cur = nxt;
        q0 += nk;
    }
    __builtin_amdgcn_s_waitcnt(vmcnt_imm(0));  // the surplus copies have landed before the workgroup ends
}

// Down projection: adds the pieces of each split leftover tile in piece order (fixed, so the result does not
// depend on timing) and scatters the fp16 rows to expert_out. Workgroup (g, rb) takes rows [rb * kFixRows, +kFixRows) of leftover tile
// j = g / 8 of XCD x = g % 8; piece pc of that tile is in the partial slot of workgroup (j * S + pc) * 8 + x of the
// tiled launch, whose grid had nloc workgroups per XCD. The tile is found as the tiled kernel finds it, from
// offsets (each wave scans the experts 64 at a time).
__global__ __launch_bounds__(kFixThreads) void ffn_tiled_fixup_kernel(TiledArgs p, int nloc) {
    constexpr int nrb = kBM / kFixRows;
    const int rb = static_cast<int>(blockIdx.x) % nrb, g = static_cast<int>(blockIdx.x) / nrb;
    const int x = g % kXcds, j = g / kXcds;
    const int lane = lane_id();
    auto tiles_of = [&](int e) {
        return e < p.E ? (p.offsets[e + 1] - p.offsets[e] + kBM - 1) / kBM * p.ntiles_n : 0;
    };
    int total = 0;
    for (int base = 0; base < p.E; base += kWave) {
        int v = tiles_of(base + lane);
#pragma unroll
        for (int d = 1; d < kWave; d <<= 1) v += __shfl_xor(v, d, kWave);
        total += v;
    }
    const XcdSched xs = xcd_sched(x, total, nloc, (p.kdim + kBK - 1) / kBK, 1);
    if (xs.S < 2 || j >= xs.L) return;
    const int t = xs.base + xs.R * nloc + j;
    // expert e with prefix(e) <= t < prefix(e) + tiles(e), prefix(e) = tiles of the experts before e
    int e = -1, before = 0, carry = 0;
    for (int base = 0; base < p.E && e < 0; base += kWave) {
        const int te = tiles_of(base + lane);
        int incl = te;
#pragma unroll
        for (int d = 1; d < kWave; d <<= 1) {
            const int v = __shfl_up(incl, d, kWave);
            if (lane >= d) incl += v;
        }
        const uint64_t hit = __ballot(te > 0 && carry + incl - te <= t && t < carry + incl);
        if (hit) {
            const int l = __builtin_ctzll(hit);
            e = base + l;
            before = carry + __shfl(incl - te, l, kWave);
        }
        carry += __shfl(incl, kWave - 1, kWave);
    }
    const int mt_count = (p.offsets[e + 1] - p.offsets[e] + kBM - 1) / kBM;
    const int local = t - before, nt = local / mt_count, mt = local - nt * mt_count;
    const int off = p.offsets[e], rows = min(kBM, p.offsets[e + 1] - off - mt * kBM);
    const float* part0 = p.partial + static_cast<size_t>(j * xs.S * kXcds + x) * (kBM * kBN);
    const size_t pstride = static_cast<size_t>(kXcds) * (kBM * kBN);  // next piece: li + 1
    const int tid = static_cast<int>(threadIdx.x);
    // 64 threads per row, 4 consecutive output columns each; 4 rows per thread, loaded together
    constexpr int kRows = kFixRows / (kFixThreads / 64);
    const int c = (tid % 64) * 4, r0 = rb * kFixRows + tid / 64;
    const float* src = part0 + r0 * kBN + c;
    f32x4 v[kRows];
#pragma unroll
    for (int u = 0; u < kRows; ++u) v[u] = *reinterpret_cast<const f32x4*>(src + u * (kFixThreads / 64) * kBN);
#pragma unroll 2
    for (int pc = 1; pc < xs.S; ++pc)
#pragma unroll
        for (int u = 0; u < kRows; ++u)
            v[u] += *reinterpret_cast<const f32x4*>(src + pc * pstride + u * (kFixThreads / 64) * kBN);
    const int col = nt * kBN + c;
#pragma unroll
    for (int u = 0; u < kRows; ++u) {
        const int r = r0 + u * (kFixThreads / 64);
        if (r >= rows || col >= p.H) continue;
        const uint32_t lo = f32_to_f16_bits(v[u][0]) | (static_cast<uint32_t>(f32_to_f16_bits(v[u][1])) << 16);
        const uint32_t hi = f32_to_f16_bits(v[u][2]) | (static_cast<uint32_t>(f32_to_f16_bits(v[u][3])) << 16);
        const int slot = p.sorted_slot[off + mt * kBM + r];
        *reinterpret_cast<uint2*>(p.out + static_cast<size_t>(slot) * p.H + col) = make_uint2(lo, hi);
    }
}

// Persistent grid: at most the workgroups the device holds at once, a multiple of the XCD count. SPLIT (the down
// projection): with p.split set, the leftover tiles are split over k and the fix-up kernel follows.
template <int EPI, bool SPLIT, bool KT>
hipError_t launch_tiled(TiledArgs p, int grid, const char* name, hipStream_t stream) {
    const void* fn = reinterpret_cast<const void*>(&ffn_tiled_kernel<EPI, SPLIT, KT>);
    const int lds = tiled_lds_bytes(p.E, EPI == kScatter);
    const int resident = resident_workgroups(fn, kThreads, lds);
    if (resident > 0 && resident < grid) grid = resident;
    grid = grid / kXcds * kXcds;
    if (grid < kXcds) grid = kXcds;
    // the leftover round is sized by the workgroups per XCD, so a split needs the grid to be all resident; each
    // workgroup owns one partial slot
    p.split = (SPLIT && p.split && resident > 0 && grid <= kMaxParts) ? 1 : 0;
    {
        TraceScope trace(name, stream);
        ffn_tiled_kernel<EPI, SPLIT, KT><<<grid, kThreads, lds, stream>>>(p);
    }
    hipError_t err = hipGetLastError();
    if (err != hipSuccess || !p.split) return err;
    {
        TraceScope trace("moe_ffn_down_fixup", stream);
        ffn_tiled_fixup_kernel<<<grid * (kBM / kFixRows), kFixThreads, 0, stream>>>(p, grid / kXcds);
    }
    return hipGetLastError();
}

}  // namespace

// Both k extents need at least two stages (the ring runs two ahead) and the tile table must fit in the LDS left
// over by the ring.
bool tiled_shape_supported(int64_t H, int64_t E, int64_t I) {
    if (H % 32 != 0 || I % 32 != 0 || H <= kBK || I <= kBK) return false;
    return tiled_lds_bytes(static_cast<int>(E), true) <= kLdsMax;
}
// The buffer offsets are 32-bit: gathered x rows (T*H*2 bytes), one expert's weights (3*I*H*2) and the sorted
// slots (T*K*4) must stay below 2 GiB. The down projection addresses hidden per tile, so T*K*I has no such bound.
bool tiled_size_supported(int64_t T, int64_t H, int64_t K, int64_t I) {
    const int64_t lim = int64_t(1) << 31;
    return T * H * 2 < lim && 3 * I * H * 2 < lim && T * K * 4 < lim && static_cast<int64_t>(kBM) * I * 2 < lim;
}
bool tiled_supported(int64_t T, int64_t H, int64_t E, int64_t K, int64_t I) {
    return tiled_shape_supported(H, E, I) && tiled_size_supported(T, H, K, I);
}
hipError_t prepare_ffn_tiled() {
    for (const void* fn : {reinterpret_cast<const void*>(&ffn_tiled_kernel<kSwiGLU, false, false>),
                           reinterpret_cast<const void*>(&ffn_tiled_kernel<kScatter, false, false>),
                           reinterpret_cast<const void*>(&ffn_tiled_kernel<kScatter, true, false>),
                           reinterpret_cast<const void*>(&ffn_tiled_kernel<kSwiGLU, false, true>),
                           reinterpret_cast<const void*>(&ffn_tiled_kernel<kScatter, false, true>),
                           reinterpret_cast<const void*>(&ffn_tiled_kernel<kScatter, true, true>)}) {
        const hipError_t err = ensure_lds_limit(fn, kLdsMax);
        if (err != hipSuccess) return err;
    }
    return hipSuccess;
}
int tiled_block_threads() { return kThreads; }
// The down projection splits leftover tiles into pieces of at least two k-stages (so only when I / kBK >= 4), and
// only when its tiles (bounded by tiled_down_grid) fill at most kSplitMaxRounds rounds of kMaxParts workgroups
// (one per CU on MI355X); a piece writes the partial slot of its workgroup, and the launch has at most
// min(kMaxParts, tiled_down_grid) workgroups.
bool tiled_down_splits(int T, int E, int K, int H, int I) {
    const int rounds = (tiled_down_grid(T, E, K, H) + kMaxParts - 1) / kMaxParts;
    return (I + kBK - 1) / kBK >= 4 && rounds <= kSplitMaxRounds;
}
size_t tiled_partial_bytes(int T, int H, int E, int K, int I) {
    if (!tiled_down_splits(T, E, K, H, I)) return 0;
    const int slots = min(kMaxParts, tiled_down_grid(T, E, K, H));
    return static_cast<size_t>(slots) * kBM * kBN * sizeof(float);
}
int tiled_rows_per_tile() { return kBM; }
// Upper bound on the tile count (sum over experts of ceil(rows_e / kBM) <= ceil(T*K / kBM) + E), rounded up to
// a multiple of the XCD count so that the XCD-contiguous remap in the kernel is a bijection on [0, grid).
int tiled_grid(int T, int E, int K, int ntiles_n) {
    const int m_bound = (T * K + kBM - 1) / kBM + E;
    const int g = m_bound * ntiles_n;
    return (g + kXcds - 1) / kXcds * kXcds;
}
int tiled_gateup_grid(int T, int E, int K, int I) { return tiled_grid(T, E, K, (I + 127) / 128); }
int tiled_down_grid(int T, int E, int K, int H) { return tiled_grid(T, E, K, (H + kBN - 1) / kBN); }

hipError_t launch_ffn_tiled(const uint16_t* x, const uint16_t* expert_weights, uint16_t* expert_out,
                            const FfnWorkspace& ws, int T, int H, int E, int K, int I, hipStream_t stream,
                            bool allow_split) {
    TiledArgs p{};
    p.sorted_slot = ws.sorted_slot;
    p.offsets = ws.offsets;
    p.w = expert_weights;
    p.T = T;
    p.E = E;
    p.K = K;
    p.H = H;
    p.I = I;
    p.act = x;
    p.out = ws.hidden;
    p.kdim = H;
    p.ndim = I;
    p.ntiles_n = (I + 127) / 128;
    p.gather = 1;
    p.partial = ws.partial;
    // an odd multiple of 32 along the reduction runs the KT instantiation, which clears the last stage's tail
    const hipError_t err = H % kBK != 0
                               ? launch_tiled<kSwiGLU, false, true>(p, tiled_gateup_grid(T, E, K, I), "moe_ffn_gateup_swiglu", stream)
                               : launch_tiled<kSwiGLU, false, false>(p, tiled_gateup_grid(T, E, K, I), "moe_ffn_gateup_swiglu", stream);
    if (err != hipSuccess) return err;
    p.act = ws.hidden;
    p.out = expert_out;
    p.kdim = I;
    p.ndim = H;
    p.ntiles_n = (H + kBN - 1) / kBN;
    p.gather = 0;
    p.split = (allow_split && tiled_down_splits(T, E, K, H, I) && ws.partial != nullptr) ? 1 : 0;
    const int dgrid = tiled_down_grid(T, E, K, H);
    if (I % kBK != 0) {
        if (p.split) return launch_tiled<kScatter, true, true>(p, dgrid, "moe_ffn_down", stream);
        return launch_tiled<kScatter, false, true>(p, dgrid, "moe_ffn_down", stream);
    }
    if (p.split) return launch_tiled<kScatter, true, false>(p, dgrid, "moe_ffn_down", stream);
    return launch_tiled<kScatter, false, false>(p, dgrid, "moe_ffn_down", stream);
}

}  // namespace moe
