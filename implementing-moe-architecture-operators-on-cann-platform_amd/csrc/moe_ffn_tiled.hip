// moe_ffn_tiled.hip -- LDS-tiled schedule of the MoeExpertFFN grouped GEMMs (many rows per expert, prefill).
//
// Reference: op_kernel/moe_expert_ffn.cpp (ComputeSwiGLU :265-333, ComputeDownProj :339-394, scatter :250-257);
// oracle: tests/moe_cpu_sim.cpp:245-296 (W_gate, W_up [I, H]; W_down [H, I]).
//
// With ~1000 rows per expert (T = 8192, K = 2, E = 16) the GEMMs have an arithmetic intensity of ~1500 flop/B
// against HBM, far above the MFMA ridge. Both are "NT": activation rows and weight rows are contiguous along the
// reduction dim k. Measured on MI355X with stripped copies of this kernel: its global loads alone take ~44% of
// its time (12 TB/s from L2), its MFMAs alone ~32%, but LDS stores + fragment reads + MFMAs without any global
// load already ~82%. Per 64-k stage a CU moves 256 KB through LDS against 2048 MFMA cycles per SIMD, and the two
// overlap poorly: the LDS side, not the memory system, is what a faster schedule has to shrink.
//   macro tile   256 activation rows x 256 weight rows x 64 k per stage; 8 waves (2 x 4), each a 128 x 64
//                sub-tile (8 x 4 v_mfma_f32_16x16x32_f16 tiles, 128 fp32 accumulators per lane: with 256 per
//                lane the accumulators plus the loop's other live values exceed one wave's register file and
//                the compiler shuffles them between register files every iteration)
//   pipeline     the next stage is copied straight from global memory into the other LDS buffer
//                (global_load_lds_dwordx4: no staging registers, no LDS store instructions) while the current
//                stage is multiplied; two LDS stages, one barrier per stage. The barrier carries no release
//                fence: one would wait for the copies in flight (vmcnt(0)) before the MFMAs are done. 7-8 %
//                faster than staging through registers.
//   LDS layout   unpadded 128-byte rows of 8 granules of 16 B; granule g of row r is stored at g ^ ((r >> 1) & 7),
//                so the 16 rows one ds_read_b128 touches (same logical granule) spread over all banks
//   gate/up      the 256 weight rows of a tile are, per wave quarter, 32 W_gate rows and the matching 32 W_up
//                rows, so each wave holds gate and up of the same (row, i) and applies SwiGLU in registers,
//                writing fp16 hidden rows
//   down         weight rows are W_down rows (output columns); the epilogue writes expert_out[slot] directly
//   scheduling   tiles are (expert, n-tile, m-tile) with m fastest, numbered from the per-expert row counts
//                at run time; the grid is an upper bound and surplus workgroups exit. Workgroups are dispatched
//                round-robin over the 8 XCDs, so the linear tile order is remapped to give each XCD a
//                contiguous range: the m-tiles that share a weight tile then share that XCD's L2.
// Rows past an expert's count are clamped to its last row on load and masked on store.

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
constexpr int kLdsBytes = kNStage * kStageHalfs * 2;
constexpr int kXcds = 8;

enum Epilogue { kSwiGLU = 0, kScatter = 1 };

struct TiledArgs {
    const uint16_t* act;         // x [T, H] (gate/up, gathered) or hidden [T*K, I] (down)
    const int32_t* sorted_slot;
    const int32_t* offsets;
    const uint16_t* w;           // expert_weights
    uint16_t* out;               // hidden or expert_out
    int E, K, H, I;
    int kdim;                    // H or I
    int ndim;                    // I (gate/up: tile covers 128 i of gate and up) or H (down)
    int ntiles_n;                // n-tiles per expert
    int gather;                  // gate/up: activation row r -> x[sorted_slot[r] / K]
};

// Barrier of the copy ring. The only LDS writes of the main loop are this wave's direct-to-LDS copies, which the
// caller's explicit vmcnt wait covers, and every fragment read of the stage has fed an MFMA before the wave gets
// here. A workgroup-scope release fence would also wait for the copies still in flight (vmcnt(0)).
__device__ __forceinline__ void ring_barrier() {
    __builtin_amdgcn_sched_barrier(0);
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
    __builtin_amdgcn_sched_barrier(0);
}

// Linear tile -> (expert, m-tile, n-tile); false when t is past the last tile.
__device__ __forceinline__ bool find_tile(const TiledArgs& p, int t, int* e_out, int* mt_out, int* nt_out,
                                          int* off_out, int* ne_out) {
    int base = 0;
    for (int e = 0; e < p.E; ++e) {
        const int off = p.offsets[e];
        const int ne = p.offsets[e + 1] - off;
        const int mtiles = (ne + kBM - 1) / kBM;
        const int tiles = mtiles * p.ntiles_n;
        if (t < base + tiles) {
            const int local = t - base;
            *e_out = e;
            *nt_out = local / mtiles;
            *mt_out = local % mtiles;
            *off_out = off;
            *ne_out = ne;
            return true;
        }
        base += tiles;
    }
    return false;
}

template <int EPI>
__global__ __launch_bounds__(kThreads) void ffn_tiled_kernel(TiledArgs p) {
    extern __shared__ __align__(16) uint16_t lds[];
    // XCD-contiguous remap of the dispatch order
    const int G = static_cast<int>(gridDim.x);
    const int per_xcd = (G + kXcds - 1) / kXcds;
    const int b = static_cast<int>(blockIdx.x);
    const int t = (b % kXcds) * per_xcd + b / kXcds;
    int e, mt, nt, off, ne;
    if (!find_tile(p, t, &e, &mt, &nt, &off, &ne)) return;

    const int tid = static_cast<int>(threadIdx.x);
    const int wave = __builtin_amdgcn_readfirstlane(tid / kWave);
    const int lane = lane_id();
    const int row16 = lane & 15, kg = lane >> 4;
    const int wm = wave >> 2, wn = wave & 3;  // 2 x 4 waves: rows wm*128.., weight rows wn*64..
    const int m0 = mt * kBM;
    const size_t ebase = static_cast<size_t>(e) * 3 * static_cast<size_t>(p.I) * p.H;

    // direct-to-LDS plan: per stage and operand, wave w issues 4 instructions j, each filling 8 whole LDS rows
    // r = (4 w + j) * 8 + lane / 8 (128 B each); lane fetches global granule (lane % 8) ^ ((r >> 1) & 7)
    uint32_t aoff[4], boff[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int r = (wave * 4 + j) * 8 + (lane / 8);
        const int gq = (lane % 8) ^ ((r >> 1) & 7);
        const int m = min(m0 + r, ne - 1);
        const uint32_t src = p.gather ? static_cast<uint32_t>(p.sorted_slot[off + m] / p.K) : static_cast<uint32_t>(off + m);
        aoff[j] = src * static_cast<uint32_t>(p.kdim) + gq * 8;
        if (EPI == kSwiGLU) {
            const int quarter = r >> 6, sub = r & 63;
            const int ic = min(nt * 128 + quarter * 32 + (sub & 31), p.I - 1);
            boff[j] = (sub < 32 ? 0u : static_cast<uint32_t>(p.I) * p.H) + static_cast<uint32_t>(ic) * p.H + gq * 8;
        } else {
            const int n = min(nt * kBN + r, p.H - 1);
            boff[j] = 2u * static_cast<uint32_t>(p.I) * p.H + static_cast<uint32_t>(n) * p.I + gq * 8;
        }
    }
    const uint16_t* abase = p.act;
    const uint16_t* wbase = p.w + ebase;

    f32x4 acc[8][4];
    auto issue_stage = [&](int ks) {
        const int k0 = ks * kBK;
        uint16_t* sa = lds + (ks % kNStage) * kStageHalfs;
        uint16_t* sb = sa + kBM * kPitch;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            __builtin_amdgcn_global_load_lds((const __attribute__((address_space(1))) void*)(abase + aoff[j] + k0),
                                             (__attribute__((address_space(3))) void*)(sa + (wave * 4 + j) * 8 * kPitch), 16, 0, 0);
            __builtin_amdgcn_global_load_lds((const __attribute__((address_space(1))) void*)(wbase + boff[j] + k0),
                                             (__attribute__((address_space(3))) void*)(sb + (wave * 4 + j) * 8 * kPitch), 16, 0, 0);
        }
    };
    auto mma_stage = [&](int ks, bool first) {
        const int buf = ks % kNStage;
        const int sw = (row16 >> 1) & 7;
        const uint16_t* sa = lds + buf * kStageHalfs + (wm * 128 + row16) * kPitch;
        const uint16_t* sb = lds + buf * kStageHalfs + (kBM + wn * 64 + row16) * kPitch;
#pragma unroll
        for (int kk = 0; kk < kBK / 32; ++kk) {
            const int gran = ((kk * 4 + kg) ^ sw) * 8;
            f16x8 af[8];
#pragma unroll
            for (int i = 0; i < 8; ++i) af[i] = *reinterpret_cast<const f16x8*>(sa + i * 16 * kPitch + gran);
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const f16x8 bf = *reinterpret_cast<const f16x8*>(sb + j * 16 * kPitch + gran);
#pragma unroll
                for (int i = 0; i < 8; ++i)
                    acc[i][j] = mfma16x16x32(af[i], bf, first && kk == 0 ? f32x4{0.f, 0.f, 0.f, 0.f} : acc[i][j]);
            }
        }
    };

    // two LDS stages: stage s + 1 is copied into the other buffer while stage s is multiplied
    const int nstages = p.kdim / kBK;
    issue_stage(0);
    __builtin_amdgcn_s_waitcnt(vmcnt_imm(0));  // this wave's copies of stage 0 are in LDS
    ring_barrier();                            // and every wave's
    if (nstages > 1) issue_stage(1);
    mma_stage(0, true);  // the accumulators start from an inline zero, so they are never VGPR-initialised
    if (nstages > 1) {
        __builtin_amdgcn_sched_barrier(0);  // keep the copy wait after every MFMA of the stage
        __builtin_amdgcn_s_waitcnt(vmcnt_imm(0));
        ring_barrier();
        for (int s = 1; s + 1 < nstages; ++s) {
            issue_stage(s + 1);  // into the buffer stage s - 1 used: the barrier above ended its reads
            mma_stage(s, false);
            __builtin_amdgcn_sched_barrier(0);
            __builtin_amdgcn_s_waitcnt(vmcnt_imm(0));
            ring_barrier();
        }
        mma_stage(nstages - 1, false);
    }

    // ---- epilogue: acc[i][j] lane holds D[m = 4*kg + r][n = row16] of sub-tile (i, j) ----
#pragma unroll
    for (int i = 0; i < 8; ++i)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int m = m0 + wm * 128 + i * 16 + kg * 4 + r;
            if (m >= ne) continue;
            if (EPI == kSwiGLU) {
                uint16_t* dst = p.out + static_cast<size_t>(off + m) * p.I;
#pragma unroll
                for (int j = 0; j < 2; ++j) {
                    const int col = nt * 128 + wn * 32 + j * 16 + row16;
                    if (col < p.I) dst[col] = f32_to_f16_bits(swiglu_f32(acc[i][j][r], acc[i][j + 2][r]));
                }
            } else {
                uint16_t* dst = p.out + static_cast<size_t>(p.sorted_slot[off + m]) * p.H;
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const int col = nt * kBN + wn * 64 + j * 16 + row16;
                    if (col < p.H) dst[col] = f32_to_f16_bits(acc[i][j][r]);
                }
            }
        }
}

template <int EPI>
hipError_t launch_tiled(const TiledArgs& p, int grid, hipStream_t stream) {
    const hipError_t attr = ensure_lds_limit(reinterpret_cast<const void*>(&ffn_tiled_kernel<EPI>), kLdsBytes);
    if (attr != hipSuccess) return attr;
    ffn_tiled_kernel<EPI><<<grid, kThreads, kLdsBytes, stream>>>(p);
    return hipGetLastError();
}

}  // namespace

bool tiled_supported(int H, int I) { return H % kBK == 0 && I % kBK == 0; }
int tiled_block_threads() { return kThreads; }
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
                            const FfnWorkspace& ws, int T, int H, int E, int K, int I, hipStream_t stream) {
    TiledArgs p{};
    p.sorted_slot = ws.sorted_slot;
    p.offsets = ws.offsets;
    p.w = expert_weights;
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
    hipError_t err;
    {
        TraceScope trace("moe_ffn_gateup_swiglu", stream);
        err = launch_tiled<kSwiGLU>(p, tiled_gateup_grid(T, E, K, I), stream);
    }
    if (err != hipSuccess) return err;
    p.act = ws.hidden;
    p.out = expert_out;
    p.kdim = I;
    p.ndim = H;
    p.ntiles_n = (H + kBN - 1) / kBN;
    p.gather = 0;
    {
        TraceScope trace("moe_ffn_down", stream);
        err = launch_tiled<kScatter>(p, tiled_down_grid(T, E, K, H), stream);
    }
    return err;
}

}  // namespace moe
