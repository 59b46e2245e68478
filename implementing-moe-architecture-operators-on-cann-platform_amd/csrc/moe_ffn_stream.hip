// moe_ffn_stream.hip -- weight-streaming schedule of the MoeExpertFFN grouped GEMMs (few rows per expert).
//
// Reference: op_kernel/moe_expert_ffn.cpp (ComputeSwiGLU :265-333, ComputeDownProj :339-394, scatter :250-257);
// oracle: tests/moe_cpu_sim.cpp:245-296 (W_gate, W_up [I, H]; W_down [H, I]).
//
// With few rows per expert (decode: T = 128, K = 2, E = 16 -> ~16 rows) each weight byte serves only those
// rows, so the GEMMs are bound by streaming E*3*I*H*2 bytes from HBM once. What the MI355X measurements behind
// this design showed (pure load kernels reading the 1.07 GB of decode gate/up weights at the real [E, 3I, H]
// layout, 8 waves per CU, 16 KB in flight per wave):
//   * the shape of one load instruction decides the rate. Loading straight into the MFMA operand order puts
//     16 weight rows x 64 B (half a 128-B line each) in every instruction and tops out at ~5.8 TB/s with any
//     cache policy (5.3 TB/s non-temporal). Whole lines do better only when also non-temporal: 8 rows x 128 B
//     6.5 TB/s, 1 row x 1 KB 7.0 TB/s; without the non-temporal hint every shape stays at ~5.9 TB/s;
//   * so each 64-k column block of a tile is loaded as two non-temporal 8-row x 128-B instructions and each
//     wave re-lays it into the MFMA order through 2 KB of its own LDS (one write, one read per 16 B; 6.85 TB/s
//     in the pure-load kernel with the re-layout included). Wider shapes need more LDS per wave than is left
//     beside the 128 KB activation stage;
//   * activation loads issued through the same vector-memory queue cost 10-40%: loads retire in order and the
//     L2-served traffic competes with the HBM stream -> activations are staged in LDS once per workgroup;
//   * all waves walking the rows in the same k order hit the same address-mod-4KB at the same time (rows are
//     4 KB / 16 KB apart): each wave starts at a different column block (rotation);
//   * register spills in the loop are fatal: scratch reloads also wait on the vector-memory counter and drain
//     the weight ring -> 8 waves per workgroup, no spills (checked with -Rpass-analysis=kernel-resource-usage);
//   * what did not pay: issuing the next unit's first loads before this unit's epilogue (slower by 3%), and
//     pinning the load / MFMA interleave of the ring with scheduling barriers (slower by 1.5%).
//
// Work unit = one expert e, one K-range [k0, k0 + kc) and one column group (8 waves x 16 or 32 weight rows).
// The grid is persistent: as many 8-wave workgroups as the GPU holds at once, each taking a contiguous run of
// units ordered (expert, K-range, column group) with the column group fastest. Per unit:
//   1. gate/up finds the expert's rows itself: two ballot scans of expert_ids (count, then rank) give the
//      expert's first sorted row and the slots of the current pass, so no separate permute kernel runs; the
//      workgroup holding the expert's first column group also writes offsets[e] and the expert's sorted_slot
//      entries for the down kernel. Down reads them.
//   2. unless the previous unit of the workgroup had the same expert, K-range and pass, the workgroup copies
//      the K-range of the pass's activation rows (up to 32; x rows gathered by slot / K for gate/up, SwiGLU rows
//      for down) into LDS, then one barrier;
//   3. each wave streams two 16-row weight tiles (gate/up: W_gate and W_up rows n0..n0+15; down: W_down rows
//      n0..n0+31) through a register ring of D/2 column blocks (D k-steps of 32), starting at its own rotated
//      block; per block: the four whole-line loads go through the wave's LDS re-layout buffer, activation
//      fragments come from the LDS stage (ds_read_b128), v_mfma_f32_16x16x32_f16 (fp32 accumulation).
//      With kc = 32 (D = 1) the loads go straight into the MFMA order instead (register ring of D k-steps);
//   4. epilogue in registers: gate/up -> hidden = silu(gate) * up (fp32) -> fp16 workspace row; gate/up over
//      several K-ranges (an H whose 32 rows do not fit LDS whole) -> fp32 gate and up partial sums, which
//      gateup_reduce_kernel adds in K-range order before the SwiGLU;
//      down with one K-range -> expert_out[slot] fp16 (the scatter back to [T, K, H] order);
//      down with several K-ranges -> fp32 partial sums, added in a fixed order by down_reduce_kernel (no atomics,
//      deterministic). Letting the last of the nsplit workgroups of an (expert, column group) add them instead
//      (a device-scope arrival counter, partials written and read with device-scope accesses) was measured
//      slower at decode: 121.6 us for down against 104 + 6.5 us for down + reduce.
// A workgroup per unit instead (1024 short workgroups at decode) re-stages the activations for every unit and
// lets every CU's weight stream run dry between workgroups: the persistent grid is 9% faster on gate/up.
// An expert with more than 32 rows takes several passes, each re-streaming the weights: this schedule is
// chosen only when the average number of rows per expert is small.
// LDS: row r of the staged K-range at r * (kc + 8) halfs (16 B of padding per row puts the 16 rows read by one
// ds_read_b128 in different banks), then the eight 2 KB re-layout buffers.

#include <cmath>

#include "moe_device.h"
#include "moe_launch.h"

namespace moe {

namespace {

constexpr int kWaves = 8;                 // streaming waves per workgroup
constexpr int kThreads = kWaves * kWave;  // 512
constexpr int kMaxRows = 32;              // activation rows per pass (two 16-row MFMA tiles)
constexpr int kWideRows = 128;            // wide kernel: activation rows per pass (eight 16-row MFMA tiles)
// A pass over at most kWideRowsLow rows (an expert's last pass, or its only one) runs without the eight-tile path
// and then fits a ring of kWideDepthLow k-steps in the registers. Up to kWideLowMaxRows rows per expert on average
// the wide kernels run such passes; above it most experts need 128-row passes, and the workgroups of the experts
// that do not finish early and leave the tail to the slower passes. The FFN at H = 2048, E = 16, K = 2, I = 8192
// (us, 128-row passes only / with the 64-row passes): T = 256 (32 rows per expert) 330.4 / 304.9, T = 384 (48)
// 352.6 / 325.0, T = 448 (56) 354.5 / 334.7; at T = 464 (58) an earlier build of the 64-row passes took 368.0
// against 359.6. Mixtral's H = 4096, E = 8, I = 14336: T = 192 (48) 576.1 / 558.5, T = 224 (56) 612.0 / 598.8.
// Running every pass of up to 64 rows that way (an expert of 65 rows in two passes) streams twice the weights of
// every expert above 64 rows: 466.0 us at T = 464.
constexpr int kWideRowsLow = 64;
constexpr int kWideDepthLow = 8;
constexpr int64_t kWideLowMaxRows = 56;
// Ring depth of the wide kernels (k-steps in flight per wave), whatever the narrow kernels use: with 8 the wide
// gate/up kernel spilled 33 registers in its loop and ran 8-12 % slower (T = 128, H = 4096, E = 8, I = 14336:
// 390 against 358 us; T = 512, H = 2048, E = 16, I = 8192: 281 against 251 us).
constexpr int kWideDepth = 4;
constexpr int64_t kWideMinRows = 32;      // average rows per expert from which the wide kernel runs
constexpr int kLdsMax = 160 * 1024 - 1024;  // gfx950 LDS per workgroup, less 1 KB for the static arrays

constexpr int kTbBytes = kWaves * 2048;     // per-wave 2 KB re-layout buffers of the full-line ring

// kGatePartial: gate/up over one K-range of a split H, writing fp32 gate and up sums that gateup_reduce_kernel adds
// (in split order) before the SwiGLU
enum Epilogue { kSwiGLU = 0, kScatter = 1, kPartial = 2, kGatePartial = 3 };
__host__ __device__ constexpr bool gate_up(int epi) { return epi == kSwiGLU || epi == kGatePartial; }

struct StreamArgs {
    const uint16_t* act;          // activation rows: x [T, H] (gate/up) or hidden [T*K, I] (down)
    const int32_t* sorted_slot;   // [T*K]
    const int32_t* offsets;       // [E+1]
    const uint16_t* w;            // expert_weights [E, 3I, H]
    uint16_t* out;                // hidden (kSwiGLU) or expert_out (kScatter); unused by the partial epilogues
    float* partial;               // fp32 [nsplit][T*K][H] (kPartial) or [nsplit][T*K][2I] (kGatePartial)
    int E, K, H, I;
    int kdim;                     // reduction extent: H (gate/up) or I (down)
    int ndim;                     // output columns: I (gate/up) or H (down)
    int kc;                       // K-range per workgroup (kdim % kc == 0, (kc / 32) % D == 0)
    int rows_cap;                 // activation rows per pass: 32, or 16 when 32 rows of kc do not fit LDS
    int nsplit;                   // kdim / kc
    int total_rows;               // T*K (partial buffer stride)
    size_t w_off;                 // first weight matrix inside an expert block: 0 (gate) or 2*I*H (down)
    size_t w1_off;                // second weight tile relative to the first: I*H (up) or 16*I (next 16 rows)
    int gather;                   // activation row r is x[sorted_slot[r] / K] (gate/up) or hidden[r] (down)
    const int32_t* ids;           // expert_ids [T*K]: gate/up finds each expert's rows by scanning them
    int S;                        // T*K
    int kchunk;                   // wide kernel: K columns staged in LDS at a time (kc % kchunk == 0)
    int32_t* offsets_out;         // gate/up writes offsets [E+1] and sorted_slot [T*K] for the down kernel
    int32_t* sorted_out;
    int32_t* slot_row_out;        // and the inverse: slot_row[slot] = sorted row, for the slots of valid ids
    uint16_t* expert_out;         // gate/up zeroes the rows of ids outside [0, E)
    int deal_active;              // deal the units of the active experts only (T*K <= E: most experts have no rows)
};

__device__ __forceinline__ void lds_barrier() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

// D k-steps on ring slots 0..D-1: activation fragments from LDS at physical step `ph`, then (REFILL) reload
// each slot with physical step `pn` + i.
template <int MT, int D, bool REFILL>
__device__ __forceinline__ void ring_batch(const uint16_t* lds, int stride, int ph, int pn, int row, int kg,
                                           const uint16_t* w0, const uint16_t* w1, f16x8 (&r0)[D], f16x8 (&r1)[D],
                                           f32x4 (&acc0)[MT], f32x4 (&acc1)[MT]) {
#pragma unroll
    for (int i = 0; i < D; ++i) {
        f16x8 a[MT];
#pragma unroll
        for (int mt = 0; mt < MT; ++mt)
            a[mt] = *reinterpret_cast<const f16x8*>(lds + (mt * 16 + row) * stride + (ph + i) * 32 + kg * 8);
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) {
            acc0[mt] = mfma16x16x32(a[mt], r0[i], acc0[mt]);
            acc1[mt] = mfma16x16x32(a[mt], r1[i], acc1[mt]);
        }
        if (REFILL) {
            r0[i] = load_f16x8(w0 + (pn + i) * 32);
            r1[i] = load_f16x8(w1 + (pn + i) * 32);
        }
    }
}

// D[m][n]: m = 4*kg + j (activation row of tile mt), n = row (weight row of the tile)
template <int MT, int EPI>
__device__ __forceinline__ void epilogue(const StreamArgs& p, const f32x4 (&acc0)[MT], const f32x4 (&acc1)[MT],
                                         int off, int ne, int mc, int n0, int split, int lane) {
    const int row = lane & 15, kg = lane >> 4;
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int m = mc + mt * 16 + kg * 4 + j;
            if (m >= ne) continue;
            if (EPI == kSwiGLU) {
                const float hv = swiglu_f32(acc0[mt][j], acc1[mt][j]);
                p.out[static_cast<size_t>(off + m) * p.ndim + n0 + row] = f32_to_f16_bits(hv);
            } else if (EPI == kGatePartial) {
                float* dst = p.partial + (static_cast<size_t>(split) * p.total_rows + off + m) * (2 * p.ndim) + n0 + row;
                dst[0] = acc0[mt][j];
                dst[p.ndim] = acc1[mt][j];
            } else if (EPI == kScatter) {
                const size_t o = static_cast<size_t>(p.sorted_slot[off + m]) * p.ndim + n0 + row;
                p.out[o] = f32_to_f16_bits(acc0[mt][j]);
                p.out[o + 16] = f32_to_f16_bits(acc1[mt][j]);
            } else {
                float* dst = p.partial + (static_cast<size_t>(split) * p.total_rows + off + m) * p.ndim + n0 + row;
                dst[0] = acc0[mt][j];
                dst[16] = acc1[mt][j];
            }
        }
}

// Whole K-range of one pass for one wave; the ring was primed by the caller at step `rot`.
template <int MT, int D, int EPI>
__device__ __forceinline__ void ring_pass(const StreamArgs& p, const uint16_t* lds, const uint16_t* w0,
                                          const uint16_t* w1, f16x8 (&r0)[D], f16x8 (&r1)[D], int rot, int off,
                                          int ne, int mc, int n0, int split, int lane) {
    const int row = lane & 15, kg = lane >> 4;
    const int nsteps = p.kc / 32;
    const int stride = p.kc + 8;
    f32x4 acc0[MT], acc1[MT];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
        acc0[mt] = f32x4{0.f, 0.f, 0.f, 0.f};
        acc1[mt] = f32x4{0.f, 0.f, 0.f, 0.f};
    }
    for (int s0 = 0; s0 < nsteps; s0 += D) {
        const int ph = s0 + rot < nsteps ? s0 + rot : s0 + rot - nsteps;
        const int pn = s0 + D + rot < nsteps ? s0 + D + rot : s0 + D + rot - nsteps;
        if (s0 + D < nsteps)
            ring_batch<MT, D, true>(lds, stride, ph, pn, row, kg, w0, w1, r0, r1, acc0, acc1);
        else
            ring_batch<MT, D, false>(lds, stride, ph, pn, row, kg, w0, w1, r0, r1, acc0, acc1);
    }
    epilogue<MT, EPI>(p, acc0, acc1, off, ne, mc, n0, split, lane);
}

// Full-line ring: a column block is 64 k of both tiles (two MFMA steps), loaded as four non-temporal
// instructions that each cover 8 whole weight rows x 128 B: tile 0 rows 0-7, tile 0 rows 8-15, tile 1 rows 0-7,
// tile 1 rows 8-15 (lane -> row lane / 8, 16 B chunk lane % 8). The wave then re-lays each tile through its own
// 2 KB of LDS into the MFMA B order (row lane % 16, chunk 4 * step + lane / 16).
// Buffer: row r, chunk c at r * 128 + ((c ^ ((r >> 1) & 7)) * 16) bytes -> conflict-free writes and reads.
__device__ __forceinline__ int tb_off(int r, int c) { return r * 64 + ((c ^ ((r >> 1) & 7)) * 8); }  // halfs

template <int CB>
__device__ __forceinline__ void line_prime(const uint16_t* const (&wr)[4], int rotb, f16x8 (&rg)[CB][4]) {
#pragma unroll
    for (int i = 0; i < CB; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) rg[i][j] = load_f16x8_stream(wr[j] + (rotb + i) * 64);
}

template <int MT, int CB, int EPI>
__device__ __forceinline__ void line_pass(const StreamArgs& p, const uint16_t* lds, uint16_t* tb,
                                          const uint16_t* const (&wr)[4], f16x8 (&rg)[CB][4], int rotb, int off,
                                          int ne, int mc, int n0, int split, int lane) {
    const int row = lane & 15, kg = lane >> 4;
    const int nblk = p.kc / 64;
    const int stride = p.kc + 8;
    const int wrow = lane >> 3, wc = lane & 7;
    f32x4 acc0[MT], acc1[MT];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
        acc0[mt] = f32x4{0.f, 0.f, 0.f, 0.f};
        acc1[mt] = f32x4{0.f, 0.f, 0.f, 0.f};
    }
    for (int b0 = 0; b0 < nblk; b0 += CB) {
#pragma unroll
        for (int i = 0; i < CB; ++i) {
            const int ph = b0 + i + rotb < nblk ? b0 + i + rotb : b0 + i + rotb - nblk;
            f16x8 bf[2][2];
#pragma unroll
            for (int m = 0; m < 2; ++m) {
                *reinterpret_cast<f16x8*>(tb + tb_off(wrow, wc)) = rg[i][2 * m];
                *reinterpret_cast<f16x8*>(tb + tb_off(8 + wrow, wc)) = rg[i][2 * m + 1];
                // the reads below take what other lanes of this wave just wrote: keep the compiler from moving
                // them above the writes (LDS operations of one wave execute in order, so no wait is needed)
                __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
                __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
                bf[m][0] = *reinterpret_cast<const f16x8*>(tb + tb_off(row, kg));
                bf[m][1] = *reinterpret_cast<const f16x8*>(tb + tb_off(row, 4 + kg));
                __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");  // reads done before the next writes
                __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
            }
            if (b0 + CB < nblk) {
                const int pn = ph + CB < nblk ? ph + CB : ph + CB - nblk;
#pragma unroll
                for (int j = 0; j < 4; ++j) rg[i][j] = load_f16x8_stream(wr[j] + pn * 64);
            }
#pragma unroll
            for (int st = 0; st < 2; ++st) {
                f16x8 a[MT];
#pragma unroll
                for (int mt = 0; mt < MT; ++mt)
                    a[mt] = *reinterpret_cast<const f16x8*>(lds + (mt * 16 + row) * stride + (2 * ph + st) * 32 + kg * 8);
#pragma unroll
                for (int mt = 0; mt < MT; ++mt) {
                    acc0[mt] = mfma16x16x32(a[mt], bf[0][st], acc0[mt]);
                    acc1[mt] = mfma16x16x32(a[mt], bf[1][st], acc1[mt]);
                }
            }
            __builtin_amdgcn_sched_barrier(0);
        }
    }
    epilogue<MT, EPI>(p, acc0, acc1, off, ne, mc, n0, split, lane);
}

// Wide passes (up to 64 or 128 activation rows, MT row tiles): the K-range is staged in LDS one chunk of kchunk
// columns (bpc column blocks of 64) at a time. The ring runs over the sequence of blocks chunk by chunk, each chunk
// in the rotated order (j + rotc) % bpc, and refills each slot with the block CB places later in the sequence
// (which may lie in the next chunk). One call multiplies the blocks of chunk c into the accumulators.
template <int MT, int CB>
__device__ __forceinline__ void line_chunk(const uint16_t* lds, uint16_t* tb, const uint16_t* const (&wr)[4],
                                           f16x8 (&rg)[CB][4], f32x4 (&acc0)[MT], f32x4 (&acc1)[MT], int c,
                                           int nchunk, int bpc, int rotc, int stride, int lane) {
    const int row = lane & 15, kg = lane >> 4;
    const int wrow = lane >> 3, wc = lane & 7;
    const int nseq = nchunk * bpc;
    for (int j0 = 0; j0 < bpc; j0 += CB) {
#pragma unroll
        for (int i = 0; i < CB; ++i) {
            int jl = j0 + i + rotc;
            jl = jl < bpc ? jl : jl - bpc;  // block of the chunk = column block of the LDS stage
            f16x8 bf[2][2];
#pragma unroll
            for (int m = 0; m < 2; ++m) {
                *reinterpret_cast<f16x8*>(tb + tb_off(wrow, wc)) = rg[i][2 * m];
                *reinterpret_cast<f16x8*>(tb + tb_off(8 + wrow, wc)) = rg[i][2 * m + 1];
                __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
                __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
                bf[m][0] = *reinterpret_cast<const f16x8*>(tb + tb_off(row, kg));
                bf[m][1] = *reinterpret_cast<const f16x8*>(tb + tb_off(row, 4 + kg));
                __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
                __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
            }
            const int sn = c * bpc + j0 + i + CB;  // the block this slot loads next
            if (sn < nseq) {
                const int cn = sn / bpc;
                int jn = sn - cn * bpc + rotc;
                jn = jn < bpc ? jn : jn - bpc;
#pragma unroll
                for (int j = 0; j < 4; ++j) rg[i][j] = load_f16x8_stream(wr[j] + (cn * bpc + jn) * 64);
            }
#pragma unroll
            for (int st = 0; st < 2; ++st) {
                f16x8 a[MT];
#pragma unroll
                for (int mt = 0; mt < MT; ++mt)
                    a[mt] = *reinterpret_cast<const f16x8*>(lds + (mt * 16 + row) * stride + (2 * jl + st) * 32 + kg * 8);
#pragma unroll
                for (int mt = 0; mt < MT; ++mt) {
                    acc0[mt] = mfma16x16x32(a[mt], bf[0][st], acc0[mt]);
                    acc1[mt] = mfma16x16x32(a[mt], bf[1][st], acc1[mt]);
                }
            }
            __builtin_amdgcn_sched_barrier(0);
        }
    }
}

// Expert e's rows by scanning ids: wave w takes the contiguous chunk w of the T*K slots.
// count: per-wave numbers of ids == e and of valid ids < e into s_eq / s_lt (the caller then barriers);
// rank:  the slots of e in ascending order get ranks 0..ne-1; those in [mc, mc + cap) go to s_rows, and with
//        `sorted` non-null every slot is written to sorted[off + rank] and off + rank to slot_row[slot].
__device__ __forceinline__ void expert_count(const StreamArgs& p, int e, int* s_eq, int* s_lt) {
    const int wave = static_cast<int>(threadIdx.x) / kWave, lane = lane_id();
    const int chunk = ((p.S + kWaves - 1) / kWaves + kWave - 1) / kWave * kWave;
    const int beg = min(p.S, wave * chunk), end = min(p.S, beg + chunk);
    int n_eq = 0, n_lt = 0;
    for (int base = beg; base < end; base += 4 * kWave) {
        int id[4];
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            const int sl = base + u * kWave + lane;
            id[u] = sl < end ? p.ids[sl] : -1;
        }
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            n_eq += __popcll(__ballot(id[u] == e));
            n_lt += __popcll(__ballot(id[u] >= 0 && id[u] < e));
        }
    }
    if (lane == 0) {
        s_eq[wave] = n_eq;
        s_lt[wave] = n_lt;
    }
}

__device__ __forceinline__ void expert_rank(const StreamArgs& p, int e, int before, int off, int mc, int cap,
                                            int* s_rows, int32_t* sorted) {
    const int wave = static_cast<int>(threadIdx.x) / kWave, lane = lane_id();
    const int chunk = ((p.S + kWaves - 1) / kWaves + kWave - 1) / kWave * kWave;
    const int beg = min(p.S, wave * chunk), end = min(p.S, beg + chunk);
    const uint64_t below = (uint64_t{1} << lane) - 1;
    int pos = before;
    for (int base = beg; base < end; base += 4 * kWave) {
        int id[4];
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            const int sl = base + u * kWave + lane;
            id[u] = sl < end ? p.ids[sl] : -1;
        }
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            const uint64_t m = __ballot(id[u] == e);
            if (id[u] == e) {
                const int rank = pos + __popcll(m & below);
                const int sl = base + u * kWave + lane;
                if (rank >= mc && rank < mc + cap) s_rows[rank - mc] = sl;
                if (sorted) {
                    sorted[off + rank] = sl;
                    p.slot_row_out[sl] = off + rank;
                }
            }
            pos += __popcll(m);
        }
    }
}

// ---- units over the active experts ----
// The persistent grid deals out only the units of experts that have rows. Dealt over all E experts, the units of
// the few experts a small batch touches fall to the few workgroups whose unit range holds them (at T = 1 and
// E = 256, 8 of 256 CUs stream all the weights). A 256-bit mask in LDS (E <= 256) names the active experts: bit
// e of s_am[e / 64]; it is read afresh where needed rather than held in registers across the unit loop.
__device__ __forceinline__ uint64_t uniform64(uint64_t v) {
    const uint32_t lo = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(v));
    const uint32_t hi = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(v >> 32));
    return (static_cast<uint64_t>(hi) << 32) | lo;
}

// gate/up: every workgroup ORs the valid ids of all T*K slots into the mask (4 id loads in flight per thread,
// then a wave OR and one 64-bit LDS OR per wave and word)
__device__ __forceinline__ void active_from_ids(const StreamArgs& p, unsigned long long* s_am) {
    const int tid = static_cast<int>(threadIdx.x), lane = lane_id();
    if (tid < 4) s_am[tid] = 0;
    lds_barrier();
    uint64_t m[4] = {0, 0, 0, 0};
    for (int base = 0; base < p.S; base += 4 * kThreads) {
        int id[4];
#pragma unroll
        for (int t = 0; t < 4; ++t) {
            const int sl = base + t * kThreads + tid;
            id[t] = sl < p.S ? p.ids[sl] : -1;
        }
#pragma unroll
        for (int t = 0; t < 4; ++t) {
            const bool valid = id[t] >= 0 && id[t] < p.E;
            const uint64_t bit = valid ? uint64_t{1} << (id[t] & 63) : 0;
#pragma unroll
            for (int w = 0; w < 4; ++w) m[w] |= (id[t] >> 6) == w ? bit : 0;
        }
    }
#pragma unroll
    for (int w = 0; w < 4; ++w) {
#pragma unroll
        for (int d = 1; d < kWave; d <<= 1) m[w] |= __shfl_xor(m[w], d, kWave);
        if (lane == 0 && m[w] != 0) atomicOr(&s_am[w], static_cast<unsigned long long>(m[w]));
    }
    lds_barrier();
}

// the down projection: the experts whose offsets (written by gate/up) enclose rows
__device__ __forceinline__ void active_from_offsets(const StreamArgs& p, unsigned long long* s_am) {
    const int tid = static_cast<int>(threadIdx.x);
    if (tid < 4 * kWave) {  // waves 0-3, one mask word each
        const int e = tid;
        const uint64_t m = __ballot(e < p.E && p.offsets[e + 1] > p.offsets[e]);
        if (tid % kWave == 0) s_am[tid / kWave] = m;
    }
    lds_barrier();
}

__device__ __forceinline__ uint64_t am_word(const unsigned long long* s_am, int w) { return uniform64(s_am[w]); }

__device__ __forceinline__ int active_count(const unsigned long long* s_am) {
    return __popcll(am_word(s_am, 0)) + __popcll(am_word(s_am, 1)) + __popcll(am_word(s_am, 2)) +
           __popcll(am_word(s_am, 3));
}

// the a-th active expert (a < active_count)
__device__ __forceinline__ int nth_active(const unsigned long long* s_am, int a) {
    for (int w = 0; w < 4; ++w) {
        const int c = __popcll(am_word(s_am, w));
        if (a < c) {
            uint64_t m = am_word(s_am, w);
            for (int i = 0; i < a; ++i) m &= m - 1;
            return w * 64 + __builtin_ctzll(m);
        }
        a -= c;
    }
    return -1;
}

// the highest active expert below e (-1 if none) and the lowest above e (-1 if none)
__device__ __forceinline__ int prev_active(const unsigned long long* s_am, int e) {
    for (int w = e >> 6; w >= 0; --w) {
        uint64_t m = am_word(s_am, w);
        if (w == (e >> 6)) m &= (uint64_t{1} << (e & 63)) - 1;
        if (m != 0) return w * 64 + 63 - __builtin_clzll(m);
    }
    return -1;
}
__device__ __forceinline__ int next_active(const unsigned long long* s_am, int e) {
    for (int w = e >> 6; w < 4; ++w) {
        uint64_t m = am_word(s_am, w);
        if (w == (e >> 6)) m &= (e & 63) == 63 ? 0 : ~((uint64_t{2} << (e & 63)) - 1);
        if (m != 0) return w * 64 + __builtin_ctzll(m);
    }
    return -1;
}

// gate/up, at an active expert e's first unit: offsets_out of e and of the experts without rows before it (all
// equal to e's offset), and for the last active expert those after it up to E (off + ne)
__device__ __forceinline__ void write_offsets(const StreamArgs& p, const unsigned long long* s_am, int e, int off,
                                              int ne) {
    const int tid = static_cast<int>(threadIdx.x);
    for (int x = prev_active(s_am, e) + 1 + tid; x <= e; x += kThreads) p.offsets_out[x] = off;
    if (next_active(s_am, e) < 0)
        for (int x = e + 1 + tid; x <= p.E; x += kThreads) p.offsets_out[x] = off + ne;
}

// Persistent grid: workgroup b takes units [b * units_per_wg, (b + 1) * units_per_wg) of E * nsplit * groups
// units, unit u -> (expert, K-range, column group) with the column group fastest. With DEAL (T*K <= E, so most
// experts have no rows) it takes units [b * per, (b + 1) * per) of the active experts' units instead, per =
// ceil(active units / grid), active unit ua -> (a-th active expert, K-range, column group); the unit's index u among
// all E experts' units still fixes its ring rotation, so the results do not depend on the deal.
template <int D, int EPI, bool DEAL>
__global__ __launch_bounds__(kThreads) void ffn_stream_kernel(StreamArgs p, int units_per_wg) {
    extern __shared__ __align__(16) uint16_t lds[];
    __shared__ int s_eq[kWaves], s_lt[kWaves];
    __shared__ int s_rows[kMaxRows];
    __shared__ unsigned long long s_am[4];
    const int wave = static_cast<int>(threadIdx.x) / kWave;
    const int lane = lane_id();
    const int tid = static_cast<int>(threadIdx.x);
    const int cols_per_wave = gate_up(EPI) ? 16 : 32;  // gate/up: 16 rows of each matrix; down: 32 rows
    const int groups = (p.ndim + kWaves * cols_per_wave - 1) / (kWaves * cols_per_wave);
    const int row = lane & 15, kg = lane >> 4;
    const int nsteps = p.kc / 32;
    const int gpr = p.kc / 8;
    const int stride = p.kc + 8;

    if (gate_up(EPI)) {
        // once per call: zero the expert_out rows of ids outside [0, E) (they belong to no expert); workgroup b
        // takes slots [b * per, (b + 1) * per), 4 id loads in flight per thread
        const int per = (p.S + static_cast<int>(gridDim.x) - 1) / static_cast<int>(gridDim.x);
        const int s_beg = min(p.S, static_cast<int>(blockIdx.x) * per), s_end = min(p.S, s_beg + per);
        for (int base = s_beg; base < s_end; base += 4 * kThreads) {
            int id[4];
#pragma unroll
            for (int t = 0; t < 4; ++t) {
                const int sl = base + t * kThreads + tid;
                id[t] = sl < s_end ? p.ids[sl] : 0;
            }
#pragma unroll
            for (int t = 0; t < 4; ++t) {
                if (id[t] >= 0 && id[t] < p.E) continue;
                u32x4* dst = reinterpret_cast<u32x4*>(p.expert_out + static_cast<size_t>(base + t * kThreads + tid) * p.H);
                for (int j = 0; j < p.H / 8; ++j) dst[j] = u32x4{0u, 0u, 0u, 0u};
            }
        }
    }

    const int upe = groups * p.nsplit;  // units per expert
    int ua_begin, ua_end;
    if constexpr (DEAL) {
        if (gate_up(EPI)) active_from_ids(p, s_am);
        else active_from_offsets(p, s_am);
        const int nact = active_count(s_am);
        const int per = (nact * upe + static_cast<int>(gridDim.x) - 1) / static_cast<int>(gridDim.x);
        ua_begin = min(nact * upe, static_cast<int>(blockIdx.x) * per);
        ua_end = min(nact * upe, ua_begin + per);
        if (gate_up(EPI) && nact == 0 && blockIdx.x == 0)  // no valid ids: every offset is 0
            for (int x = tid; x <= p.E; x += kThreads) p.offsets_out[x] = 0;
    } else {
        ua_begin = static_cast<int>(blockIdx.x) * units_per_wg;
        ua_end = min(ua_begin + units_per_wg, p.E * upe);
    }
    int cur_e = -1, off = 0, ne = 0, before = 0;          // expert whose counts are known (gate/up)
    int staged_e = -1, staged_split = -1, staged_mc = -1;  // activation rows held in LDS
    for (int ua = ua_begin; ua < ua_end; ++ua) {
        int e, u;
        if constexpr (DEAL) {
            e = nth_active(s_am, ua / upe);
            u = e * upe + ua % upe;
        } else {
            u = ua;
            e = u / upe;
        }
        const int g = u % groups;
        const int split = (u / groups) % p.nsplit;
        if (gate_up(EPI)) {
            if (e != cur_e) {
                if (cur_e >= 0) lds_barrier();  // every wave is done with the previous expert's counts and rows
                expert_count(p, e, s_eq, s_lt);
                lds_barrier();
                off = 0;
                ne = 0;
                before = 0;
#pragma unroll
                for (int w = 0; w < kWaves; ++w) {
                    off += s_lt[w];
                    ne += s_eq[w];
                    if (w < wave) before += s_eq[w];
                }
                cur_e = e;
                staged_mc = -1;
                if (g == 0 && split == 0) {
                    if constexpr (DEAL) {
                        write_offsets(p, s_am, e, off, ne);
                    } else if (tid == 0) {
                        p.offsets_out[e] = off;
                        if (e == p.E - 1) p.offsets_out[p.E] = off + ne;
                    }
                }
            }
        } else {
            off = p.offsets[e];
            ne = p.offsets[e + 1] - off;
        }
        if (ne <= 0) continue;  // uniform over the workgroup
        const int n0 = (g * kWaves + wave) * cols_per_wave;
        const bool active = n0 < p.ndim;
        const int k0 = split * p.kc;
        const size_t ebase = static_cast<size_t>(e) * 3 * static_cast<size_t>(p.I) * p.H;
        // D == 1 ring: lane (row, kg) reads weight row n0 + row, k-group kg of each k-step
        const uint16_t* w0 =
            p.w + ebase + p.w_off + static_cast<size_t>(active ? n0 + row : row) * p.kdim + k0 + kg * 8;
        const uint16_t* w1 = w0 + p.w1_off;
        const int rot = ((u * kWaves + wave) * 7 * D) % nsteps;  // a multiple of D: batches never wrap

        constexpr int CB = D / 2;  // column blocks in flight (full-line ring, D >= 2)
        constexpr int CBn = CB > 0 ? CB : 1;
        // D >= 2 ring: lane reads 16 B chunk lane % 8 of weight rows n0 + lane / 8 (+ 8) of each column block
        const uint16_t* wbase = p.w + ebase + p.w_off + static_cast<size_t>(active ? n0 : 0) * p.kdim + k0 +
                                static_cast<size_t>(lane >> 3) * p.kdim + (lane & 7) * 8;
        const uint16_t* const wr[4] = {wbase, wbase + static_cast<size_t>(8) * p.kdim, wbase + p.w1_off,
                                       wbase + p.w1_off + static_cast<size_t>(8) * p.kdim};

        for (int mc = 0; mc < ne; mc += p.rows_cap) {
            const int rows = min(p.rows_cap, ne - mc);
            f16x8 rg[CBn][4];   // D >= 2: whole-line ring (wr, column blocks)
            f16x8 r0[D], r1[D];  // D == 1: loads straight into the MFMA order (w0, w1, k-steps)
            if (active) {
                if constexpr (CB > 0) {
                    line_prime<CBn>(wr, rot / 2, rg);
                } else {
#pragma unroll
                    for (int i = 0; i < D; ++i) {
                        r0[i] = load_f16x8(w0 + (rot + i) * 32);
                        r1[i] = load_f16x8(w1 + (rot + i) * 32);
                    }
                }
            }
            if (e != staged_e || split != staged_split || mc != staged_mc) {
                if (staged_e >= 0) lds_barrier();  // every wave is done with the previous rows
                staged_e = e;
                staged_split = split;
                staged_mc = mc;
                if (gate_up(EPI)) {
                    expert_rank(p, e, before, off, mc, p.rows_cap, s_rows,
                                g == 0 && split == 0 && mc == 0 ? p.sorted_out : nullptr);
                    lds_barrier();
                }
                const int total = rows * gpr;
                for (int q0 = 0; q0 < total; q0 += 4 * kThreads) {
                    u32x4 v[4];
#pragma unroll
                    for (int t = 0; t < 4; ++t) {
                        const int q = q0 + t * kThreads + tid;
                        if (q < total) {
                            const int r = q / gpr;
                            const size_t src_row = p.gather ? static_cast<size_t>(s_rows[r] / p.K)
                                                            : static_cast<size_t>(off + mc + r);
                            v[t] = *reinterpret_cast<const u32x4*>(p.act + src_row * p.kdim + k0 + (q % gpr) * 8);
                        }
                    }
#pragma unroll
                    for (int t = 0; t < 4; ++t) {
                        const int q = q0 + t * kThreads + tid;
                        if (q < total) *reinterpret_cast<u32x4*>(lds + (q / gpr) * stride + (q % gpr) * 8) = v[t];
                    }
                }
                lds_barrier();
            }
            if (active) {
                if constexpr (CB > 0) {
                    uint16_t* tb = lds + p.rows_cap * stride + wave * 1024;
                    if (rows > 16)
                        line_pass<2, CBn, EPI>(p, lds, tb, wr, rg, rot / 2, off, ne, mc, n0, split, lane);
                    else
                        line_pass<1, CBn, EPI>(p, lds, tb, wr, rg, rot / 2, off, ne, mc, n0, split, lane);
                } else if (rows > 16) {
                    ring_pass<2, D, EPI>(p, lds, w0, w1, r0, r1, rot, off, ne, mc, n0, split, lane);
                } else {
                    ring_pass<1, D, EPI>(p, lds, w0, w1, r0, r1, rot, off, ne, mc, n0, split, lane);
                }
            }
        }
    }
}

// One wide pass of up to 128 rows (MT row tiles): for each K chunk, every wave waits for the others to finish the previous
// chunk, the workgroup stages the chunk's activation rows, and the active waves multiply it; the epilogue follows
// the last chunk. The ring was primed with the first CB blocks of chunk 0.
template <int MT, int CB, int EPI>
__device__ __forceinline__ void wide_pass(const StreamArgs& p, uint16_t* lds, uint16_t* tb, const uint16_t* const (&wr)[4],
                                          f16x8 (&rg)[CB][4], const int* s_rows, bool active, int rows, int kchunk,
                                          int rotc, int off, int ne, int mc, int n0, int split, int lane) {
    const int tid = static_cast<int>(threadIdx.x);
    const int bpc = kchunk / 64, nchunk = p.kc / kchunk;
    const int stride = kchunk + 8;
    const int gpr = kchunk / 8;  // 16-byte granules per staged row
    const int k0 = split * p.kc;
    f32x4 acc0[MT], acc1[MT];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
        acc0[mt] = f32x4{0.f, 0.f, 0.f, 0.f};
        acc1[mt] = f32x4{0.f, 0.f, 0.f, 0.f};
    }
    for (int c = 0; c < nchunk; ++c) {
        lds_barrier();  // every wave is done with the previous chunk's rows (or the previous pass's)
        const int total = rows * gpr;
        for (int q0 = 0; q0 < total; q0 += 4 * kThreads) {
            u32x4 v[4];
#pragma unroll
            for (int t = 0; t < 4; ++t) {
                const int q = q0 + t * kThreads + tid;
                if (q < total) {
                    const int r = q / gpr;
                    const size_t src_row = p.gather ? static_cast<size_t>(s_rows[r] / p.K) : static_cast<size_t>(off + mc + r);
                    v[t] = *reinterpret_cast<const u32x4*>(p.act + src_row * p.kdim + k0 + c * kchunk + (q % gpr) * 8);
                }
            }
#pragma unroll
            for (int t = 0; t < 4; ++t) {
                const int q = q0 + t * kThreads + tid;
                if (q < total) *reinterpret_cast<u32x4*>(lds + (q / gpr) * stride + (q % gpr) * 8) = v[t];
            }
        }
        lds_barrier();
        if (active) line_chunk<MT, CB>(lds, tb, wr, rg, acc0, acc1, c, nchunk, bpc, rotc, stride, lane);
    }
    if (active) epilogue<MT, EPI>(p, acc0, acc1, off, ne, mc, n0, split, lane);
}

// A 64-row pass stages chunks of twice the columns where the K-range allows (the LDS holds 128 rows of p.kchunk).
template <int ROWS>
__device__ __forceinline__ int wide_kchunk(const StreamArgs& p) {
    return ROWS <= 64 && p.kc % (2 * p.kchunk) == 0 ? 2 * p.kchunk : p.kchunk;
}

// Rotated start of wave `wave` of unit u inside each chunk, a multiple of CB (so a batch of CB blocks never wraps).
template <int CB>
__device__ __forceinline__ int wide_rotation(const StreamArgs& p, int u, int wave, int kchunk) {
    return (((u * kWaves + wave) * 7 * CB) % (p.kc / 64)) % (kchunk / 64) / CB * CB;
}

// One pass of the wide kernel over up to ROWS rows of expert e from row mc, with a ring of CB k-step pairs: primes
// the ring, ranks the pass's rows (gate/up) and multiplies them in MT-tile passes.
template <int CB, int EPI, int ROWS>
__device__ __forceinline__ void wide_rows(const StreamArgs& p, uint16_t* lds, uint16_t* tb, const uint16_t* const (&wr)[4],
                                          int* s_rows, bool active, int kchunk, int rotc, int e, int before, int off,
                                          int ne, int mc, int n0, int split, int32_t* sorted, int lane) {
    const int rows = min(ROWS, ne - mc);
    f16x8 rg[CB][4];
    if (active) line_prime<CB>(wr, rotc, rg);  // the first CB blocks of chunk 0
    if (gate_up(EPI)) {
        lds_barrier();  // every wave is done reading s_rows
        expert_rank(p, e, before, off, mc, ROWS, s_rows, sorted);
    }
    if (rows > 64) {
        if constexpr (ROWS > 64) wide_pass<8, CB, EPI>(p, lds, tb, wr, rg, s_rows, active, rows, kchunk, rotc, off, ne, mc, n0, split, lane);
    } else if (rows > 32) wide_pass<4, CB, EPI>(p, lds, tb, wr, rg, s_rows, active, rows, kchunk, rotc, off, ne, mc, n0, split, lane);
    else if (rows > 16) wide_pass<2, CB, EPI>(p, lds, tb, wr, rg, s_rows, active, rows, kchunk, rotc, off, ne, mc, n0, split, lane);
    else wide_pass<1, CB, EPI>(p, lds, tb, wr, rg, s_rows, active, rows, kchunk, rotc, off, ne, mc, n0, split, lane);
}

// The weight-streaming schedule for experts with ~32 to a few hundred rows: the same units and full-line ring as
// ffn_stream_kernel, but each pass covers up to kWideRows = 128 rows (MT = 1, 2, 4 or 8 row tiles, a ring of
// kWideDepth k-steps), so an expert's weights are streamed once per 128 rows instead of once per 32, and the
// K-range is staged in chunks of p.kchunk columns to fit 128 rows in LDS. With LOW, a pass with at most
// kWideRowsLow rows left runs as a 64-row pass with a ring of kWideDepthLow k-steps (p.kchunk a multiple of its
// batch) and chunks of twice p.kchunk columns where the K-range divides, so an expert of up to 64 rows streams its
// weights with twice the loads in flight and half the stages.
template <int EPI, bool LOW>
__global__ __launch_bounds__(kThreads) void ffn_stream_wide_kernel(StreamArgs p, int units_per_wg) {
    extern __shared__ __align__(16) uint16_t lds[];
    __shared__ int s_eq[kWaves], s_lt[kWaves];
    __shared__ int s_rows[kWideRows];
    constexpr int CB = kWideDepth / 2, CBL = kWideDepthLow / 2;
    static_assert(CB >= 1, "the wide kernel runs the full-line ring");
    const int wave = static_cast<int>(threadIdx.x) / kWave;
    const int lane = lane_id();
    const int tid = static_cast<int>(threadIdx.x);
    const int cols_per_wave = gate_up(EPI) ? 16 : 32;
    const int groups = (p.ndim + kWaves * cols_per_wave - 1) / (kWaves * cols_per_wave);
    const int total_units = p.E * p.nsplit * groups;
    const int u_begin = static_cast<int>(blockIdx.x) * units_per_wg;
    const int u_end = min(u_begin + units_per_wg, total_units);
    if (gate_up(EPI)) {
        const int per = (p.S + static_cast<int>(gridDim.x) - 1) / static_cast<int>(gridDim.x);
        const int s_beg = min(p.S, static_cast<int>(blockIdx.x) * per), s_end = min(p.S, s_beg + per);
        for (int base = s_beg; base < s_end; base += 4 * kThreads) {
            int id[4];
#pragma unroll
            for (int t = 0; t < 4; ++t) {
                const int sl = base + t * kThreads + tid;
                id[t] = sl < s_end ? p.ids[sl] : 0;
            }
#pragma unroll
            for (int t = 0; t < 4; ++t) {
                if (id[t] >= 0 && id[t] < p.E) continue;
                u32x4* dst = reinterpret_cast<u32x4*>(p.expert_out + static_cast<size_t>(base + t * kThreads + tid) * p.H);
                for (int j = 0; j < p.H / 8; ++j) dst[j] = u32x4{0u, 0u, 0u, 0u};
            }
        }
    }

    int cur_e = -1, off = 0, ne = 0, before = 0;
    for (int u = u_begin; u < u_end; ++u) {
        const int g = u % groups;
        const int split = (u / groups) % p.nsplit;
        const int e = u / groups / p.nsplit;
        if (gate_up(EPI)) {
            if (e != cur_e) {
                lds_barrier();  // every wave is done with the previous expert's counts and rows
                expert_count(p, e, s_eq, s_lt);
                lds_barrier();
                off = 0;
                ne = 0;
                before = 0;
#pragma unroll
                for (int w = 0; w < kWaves; ++w) {
                    off += s_lt[w];
                    ne += s_eq[w];
                    if (w < wave) before += s_eq[w];
                }
                cur_e = e;
                if (g == 0 && split == 0 && tid == 0) {
                    p.offsets_out[e] = off;
                    if (e == p.E - 1) p.offsets_out[p.E] = off + ne;
                }
            }
        } else {
            off = p.offsets[e];
            ne = p.offsets[e + 1] - off;
        }
        if (ne <= 0) continue;  // uniform over the workgroup
        const int n0 = (g * kWaves + wave) * cols_per_wave;
        const bool active = n0 < p.ndim;
        const int k0 = split * p.kc;
        const size_t ebase = static_cast<size_t>(e) * 3 * static_cast<size_t>(p.I) * p.H;
        const uint16_t* wbase = p.w + ebase + p.w_off + static_cast<size_t>(active ? n0 : 0) * p.kdim + k0 +
                                static_cast<size_t>(lane >> 3) * p.kdim + (lane & 7) * 8;
        const uint16_t* const wr[4] = {wbase, wbase + static_cast<size_t>(8) * p.kdim, wbase + p.w1_off,
                                       wbase + p.w1_off + static_cast<size_t>(8) * p.kdim};
        uint16_t* tb = lds + kWideRows * (p.kchunk + 8) + wave * 1024;
        const bool rank_out = g == 0 && split == 0;  // the expert's first pass writes sorted_out
        const int rotc = wide_rotation<CB>(p, u, wave, p.kchunk);
        if constexpr (!LOW) {
            // written out rather than through wide_rows: this form of the 128-row loop compiles to the faster code
            // (about 2 % on the FFN at 64 rows per expert)
            for (int mc = 0; mc < ne; mc += kWideRows) {
                const int rows = min(kWideRows, ne - mc);
                f16x8 rg[CB][4];
                if (active) line_prime<CB>(wr, rotc, rg);  // the first CB blocks of chunk 0
                if (gate_up(EPI)) {
                    lds_barrier();  // every wave is done reading s_rows
                    expert_rank(p, e, before, off, mc, kWideRows, s_rows, rank_out && mc == 0 ? p.sorted_out : nullptr);
                }
                if (rows > 64) wide_pass<8, CB, EPI>(p, lds, tb, wr, rg, s_rows, active, rows, p.kchunk, rotc, off, ne, mc, n0, split, lane);
                else if (rows > 32) wide_pass<4, CB, EPI>(p, lds, tb, wr, rg, s_rows, active, rows, p.kchunk, rotc, off, ne, mc, n0, split, lane);
                else if (rows > 16) wide_pass<2, CB, EPI>(p, lds, tb, wr, rg, s_rows, active, rows, p.kchunk, rotc, off, ne, mc, n0, split, lane);
                else wide_pass<1, CB, EPI>(p, lds, tb, wr, rg, s_rows, active, rows, p.kchunk, rotc, off, ne, mc, n0, split, lane);
            }
        } else {
            int32_t* const sorted = rank_out ? p.sorted_out : nullptr;
            for (int mc = 0; mc < ne; mc += kWideRows) {  // uniform over the workgroup
                if (ne - mc <= kWideRowsLow) {
                    const int kch = wide_kchunk<kWideRowsLow>(p);
                    wide_rows<CBL, EPI, kWideRowsLow>(p, lds, tb, wr, s_rows, active, kch,
                                                      wide_rotation<CBL>(p, u, wave, kch), e, before, off, ne, mc, n0,
                                                      split, mc == 0 ? sorted : nullptr, lane);
                    break;  // the expert's last pass
                }
                wide_rows<CB, EPI, kWideRows>(p, lds, tb, wr, s_rows, active, p.kchunk, rotc, e, before, off, ne, mc,
                                              n0, split, mc == 0 ? sorted : nullptr, lane);
            }
        }
    }
}

// The split reduce's loads: the 8 columns c.. of row `row` in splits s0 .. s0 + kSplitBatch - 1, issued together
// (split indices past the last read the last split again, always in bounds), then added into acc in split order:
// acc = ((p0 + p1) + p2) + ... whatever the batching. The adds are selects, not branches, so the compiler cannot
// move a split's loads behind its own test and wait for each split in turn.
constexpr int kSplitBatch = 4;
__device__ __forceinline__ void add_split_batch(const float* __restrict__ partial, size_t split_stride, size_t row_off,
                                                int s0, int nsplit, float (&acc)[8]) {
    f32x4 v[kSplitBatch][2];
#pragma unroll
    for (int u = 0; u < kSplitBatch; ++u) {
        const f32x4* src = reinterpret_cast<const f32x4*>(partial + static_cast<size_t>(min(s0 + u, nsplit - 1)) *
                                                                        split_stride + row_off);
        v[u][0] = src[0];
        v[u][1] = src[1];
    }
#pragma unroll
    for (int u = 0; u < kSplitBatch; ++u) {
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const float x = v[u][j / 4][j % 4];
            const float sum = s0 + u == 0 ? x : acc[j] + x;
            acc[j] = s0 + u < nsplit ? sum : acc[j];
        }
    }
}

// expert_out[sorted_slot[r], h] = fp16(((partial[0][r][h] + partial[1][r][h]) + ...)), 8 columns per thread.
// Every row r < total_rows lies inside the partial buffer and sorted_slot, so the loads go out before the
// valid-row bound is known; rows past it (ids outside [0, E)) are dropped afterwards.
__global__ __launch_bounds__(256) void down_reduce_kernel(const float* __restrict__ partial,
                                                          const int32_t* __restrict__ sorted_slot,
                                                          const int32_t* __restrict__ offsets, int E, int total_rows,
                                                          int H, int nsplit, uint16_t* __restrict__ expert_out) {
    const int vec = H / 8;
    const int64_t idx = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
    if (idx >= static_cast<int64_t>(total_rows) * vec) return;
    const int r = static_cast<int>(idx / vec);
    const int c = static_cast<int>(idx % vec) * 8;
    const int slot = sorted_slot[r];
    const int valid_rows = offsets[E];
    float acc[8];
    for (int s0 = 0; s0 < nsplit; s0 += kSplitBatch)
        add_split_batch(partial, static_cast<size_t>(total_rows) * H, static_cast<size_t>(r) * H + c, s0, nsplit, acc);
    f16x8 o;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        o[j] = static_cast<f16>(acc[j]);
        asm volatile("" ::"v"(o[j]));  // computed here, not behind the row test below
    }
    if (r < valid_rows) *reinterpret_cast<f16x8*>(expert_out + static_cast<size_t>(slot) * H + c) = o;
}

// The split reduce fused with MoeCombine, one thread per (token, 8 columns): for k ascending, expert_out row
// (t, k) = fp16 of the partials added in split order, exactly as down_reduce_kernel writes it, and
// y[t] = sum_k weights[t, k] * expert_out[t, k] with the combine kernel's fp32 arithmetic (accumulator from 0,
// k ascending, no contraction), so y is bit-identical to MoeCombine on that expert_out. Rows of ids outside
// [0, E) are the zero rows the gate/up kernel wrote, and enter the sum as zeros, as they do in MoeCombine.
// The slots are taken kKBatch at a time: their ids, sorted rows and weights are loaded together, then all
// their partials (slot_row holds a row only for valid ids; the others read row 0, in bounds, and are dropped).
constexpr int kKBatch = 2;
// hidden[r, i] = fp16(silu(gate) * up) with gate = ((g_0 + g_1) + ...) and up likewise, added in split order from
// the kGatePartial sums ([nsplit][total_rows][2 I] fp32: gate in columns [0, I), up in [I, 2 I)); 8 columns per
// thread. Rows past the valid rows (ids outside [0, E)) hold no sums and are skipped.
__global__ __launch_bounds__(256) void gateup_reduce_kernel(const float* __restrict__ partial,
                                                            const int32_t* __restrict__ offsets, int E,
                                                            int total_rows, int I, int nsplit,
                                                            uint16_t* __restrict__ hidden) {
    const int vec = I / 8;
    const int64_t idx = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
    if (idx >= static_cast<int64_t>(total_rows) * vec) return;
    const int r = static_cast<int>(idx / vec);
    const int c = static_cast<int>(idx % vec) * 8;
    if (r >= offsets[E]) return;
    const size_t stride = static_cast<size_t>(total_rows) * 2 * I;
    const size_t row_off = static_cast<size_t>(r) * 2 * I + c;
    float g[8], u[8];
    for (int s0 = 0; s0 < nsplit; s0 += kSplitBatch) {
        add_split_batch(partial, stride, row_off, s0, nsplit, g);
        add_split_batch(partial, stride, row_off + I, s0, nsplit, u);
    }
    f16x8 o;
#pragma unroll
    for (int j = 0; j < 8; ++j) o[j] = __builtin_bit_cast(_Float16, f32_to_f16_bits(swiglu_f32(g[j], u[j])));
    *reinterpret_cast<f16x8*>(hidden + static_cast<size_t>(r) * I + c) = o;
}

__global__ __launch_bounds__(256) void reduce_combine_kernel(const float* __restrict__ partial,
                                                             const int32_t* __restrict__ slot_row,
                                                             const int32_t* __restrict__ ids,
                                                             const uint16_t* __restrict__ weights, int E, int T,
                                                             int K, int H, int nsplit, uint16_t* __restrict__ expert_out,
                                                             uint16_t* __restrict__ y) {
#pragma clang fp contract(off)
    const int vec = H / 8;
    const int64_t idx = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
    if (idx >= static_cast<int64_t>(T) * vec) return;
    const int t = static_cast<int>(idx / vec);
    const int c = static_cast<int>(idx % vec) * 8;
    const size_t total_rows = static_cast<size_t>(T) * K;
    float yacc[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) yacc[j] = 0.0f;
    for (int k0 = 0; k0 < K; k0 += kKBatch) {
        bool valid[kKBatch];
        int id[kKBatch], srow[kKBatch], row[kKBatch];
        float w[kKBatch];
#pragma unroll
        for (int u = 0; u < kKBatch; ++u) {
            const int sl = t * K + min(k0 + u, K - 1);
            id[u] = ids[sl];
            srow[u] = slot_row[sl];
            w[u] = f16_bits_to_f32(weights[sl]);
        }
#pragma unroll
        for (int u = 0; u < kKBatch; ++u) {
            asm volatile("" ::"v"(srow[u]));  // loaded here with the ids, not behind a test of them
            valid[u] = k0 + u < K && id[u] >= 0 && id[u] < E;
            row[u] = valid[u] ? srow[u] : 0;
        }
        float acc[kKBatch][8];
        for (int s0 = 0; s0 < nsplit; s0 += kSplitBatch) {
#pragma unroll
            for (int u = 0; u < kKBatch; ++u)
                add_split_batch(partial, total_rows * H, static_cast<size_t>(row[u]) * H + c, s0, nsplit, acc[u]);
        }
#pragma unroll
        for (int u = 0; u < kKBatch; ++u) {
            const bool in = k0 + u < K;  // uniform; selects rather than a branch (see add_split_batch)
            f16x8 o;
#pragma unroll
            for (int j = 0; j < 8; ++j) o[j] = static_cast<f16>(valid[u] ? acc[u][j] : 0.0f);
            if (valid[u]) *reinterpret_cast<f16x8*>(expert_out + (static_cast<size_t>(t) * K + k0 + u) * H + c) = o;
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                const float sum = yacc[j] + w[u] * static_cast<float>(o[j]);
                yacc[j] = in ? sum : yacc[j];
            }
        }
    }
    f16x8 out;
#pragma unroll
    for (int j = 0; j < 8; ++j) out[j] = static_cast<f16>(yacc[j]);
    *reinterpret_cast<f16x8*>(y + static_cast<size_t>(t) * H + c) = out;
}

// K-range for one workgroup: the largest multiple of 32*D dividing kdim such that rows_cap rows of it (padded)
// fit the LDS; deepest ring first. Sets kc, D, rows_cap. allow_split marks the down projection, whose ring is at
// most 4 deep: at decode (I = 8192, 4 K-ranges of 2048) D = 4 runs it in 92.1-92.4 us against 93.6-94.0 us with
// D = 8 and 93.7-93.9 us with D = 2 (same box each); gate/up keeps D = 8.
struct StreamShape {
    int kc, d, rows_cap, nsplit;
};

StreamShape pick_shape(int kdim, bool allow_split) {
    for (int rows_cap : {kMaxRows, 16}) {
        const int kc_max = (kLdsMax - kTbBytes) / (rows_cap * 2) - 8;
        for (int d = allow_split ? 4 : 8; d >= 1; d /= 2) {
            int best = 0;
            for (int kc = 32 * d; kc <= kc_max && kc <= kdim; kc += 32 * d)
                if (kdim % kc == 0) best = kc;
            if (best > 0 && (allow_split || best == kdim)) return StreamShape{best, d, rows_cap, kdim / best};
        }
    }
    return StreamShape{0, 0, 0, 0};  // no layout: the caller reports unsupported
}

// Gate/up needs the whole of H per unit for its SwiGLU. When 32 rows of the whole H do not fit the LDS (H above
// 2272), each unit covers one K-range of H at 32 rows instead and writes fp32 gate and up sums (kGatePartial),
// which gateup_reduce_kernel adds before the SwiGLU: one more launch and 2 * nsplit * 4 bytes per (row, i) of
// traffic, where the whole-H layout holds 16 rows (an expert with more rows re-streams its weights per 16 rows;
// up to H = 4568) or none at all. The K-range is the largest multiple of 32 D dividing H, deepest ring first, and at
// least 256 columns: at H = 2336 the only split is 73 K-ranges of 32, and the FFN took 473.5 us against 183.3 us
// unsplit (T = 64, E = 16, K = 2, I = 4096).
StreamShape gateup_split_shape(int H) {
    const int kc_max = (kLdsMax - kTbBytes) / (kMaxRows * 2) - 8;
    for (int d = 8; d >= 1; d /= 2) {
        int best = 0;
        for (int kc = 32 * d; kc <= kc_max && kc <= H; kc += 32 * d)
            if (H % kc == 0 && kc >= 256) best = kc;
        if (best > 0) return StreamShape{best, d, kMaxRows, H / best};
    }
    return StreamShape{0, 0, 0, 0};
}
// Average rows per expert from which the 32-row kernel splits an H that 16 rows fit whole: below it one 16-row
// pass covers most experts and the partial sums are extra traffic. The FFN at E = 16, K = 2, I = 4096, 16-row
// passes over the whole H / split (us):
//   H = 2816 (11 K-ranges): 8 rows per expert 186.7 / 229.8, 24 rows 311.6 / 272.2
//   H = 3072 (2 K-ranges):  8 rows 202.0 / 212.1, 24 rows 339.7 / 236.1
//   H = 4096 (2 K-ranges):  8 rows 254.0 / 274.7, 24 rows 533.8 / 435.5; Mixtral's E = 8, I = 14336 at 16 rows
//                           643 / 514
constexpr int64_t kGateUpSplitMinRows = 12;
StreamShape gateup_shape(int64_t T, int H, int64_t E, int64_t K, bool allow_split) {
    const StreamShape whole = pick_shape(H, false);
    if (whole.kc > 0 && (whole.rows_cap == kMaxRows || T * K < kGateUpSplitMinRows * E)) return whole;
    const StreamShape split = allow_split ? gateup_split_shape(H) : StreamShape{0, 0, 0, 0};
    return split.kc > 0 ? split : whole;
}
// The wide kernels stage the K-range in chunks whatever its length, so their gate/up always takes the whole of H
// (no partial sums); wide_chunk(H) == 0 (H not a multiple of 128) rules the wide kernels out.
int wide_chunk(int kc, int rows, int depth);
StreamShape gateup_wide_shape(int H) {
    return wide_chunk(H, kWideRows, kWideDepth) > 0 ? StreamShape{H, kWideDepth, kWideRows, 1} : StreamShape{0, 0, 0, 0};
}

// ---- tiny batches: K-ranges that fill the grid ----
// With T*K <= E the 32-row kernels deal their units over the active experts, at most T*K of them. Where even T*K
// active experts would give fewer than kTinyUnits units, the K-range is halved until they do (down to 256
// columns; fp32 partial sums, reduced as for a long H or I): a single token's layer otherwise streamed its
// weights on 48-66 CUs at ~45 GB/s each. The FFN (unsplit / halving below 128 units / below 256 units, us):
//   H = 2048, E = 16, K = 2, I = 8192:   T = 1 56.2 / 48.4 / 47.0,  T = 2 75.4 / 75.6 / 74.0
//   H = 2048, E = 64, K = 6, I = 1408:   T = 1 43.8 / 34.9 / 37.0,  T = 2 50.4 / 47.1 / 54.6
//   H = 4096, E = 8,  K = 2, I = 14336:  T = 1 120.7 / 121.1 / 124.8
//   H = 7168, E = 256, K = 8, I = 2048:  T = 1 119.3 / 119.4 / 124.5
// (from ~200 units the reduce launch and the shorter rings cost more than the extra CUs bring).
constexpr int kTinyUnits = 128;
StreamShape tiny_split(StreamShape s, int kdim, int64_t slots, int groups, int max_d) {
    const int kc_max32 = (kLdsMax - kTbBytes) / (kMaxRows * 2) - 8;
    while (s.kc > 0 && slots * groups * s.nsplit < kTinyUnits) {
        const int kc = s.kc / 2;
        if (kc < 256 || kc % 32 != 0 || kdim % kc != 0) break;
        int d = max_d;
        while (d > 1 && kc % (32 * d) != 0) d /= 2;
        s = StreamShape{kc, d, kc <= kc_max32 ? kMaxRows : 16, kdim / kc};
    }
    return s;
}
// The K-range layouts of a call: gate/up (whole H, split H, or the wide kernels' chunked H) and down.
StreamShape stream_gateup_shape(int64_t T, int H, int64_t E, int64_t K, int I, bool wide, bool gateup_split) {
    if (wide) return gateup_wide_shape(H);
    const StreamShape s = gateup_shape(T, H, E, K, gateup_split);
    return gateup_split && T * K <= E ? tiny_split(s, H, T * K, (I + kWaves * 16 - 1) / (kWaves * 16), 8) : s;
}
StreamShape stream_down_shape(int64_t T, int H, int64_t E, int64_t K, int I, bool wide) {
    const StreamShape s = pick_shape(I, true);
    return !wide && T * K <= E ? tiny_split(s, I, T * K, (H + kWaves * 32 - 1) / (kWaves * 32), 4) : s;
}

template <int EPI>
hipError_t launch_stream_epi(const StreamArgs& p, int d, int units, hipStream_t stream) {
    const size_t lds = static_cast<size_t>(p.rows_cap) * (p.kc + 8) * sizeof(uint16_t) + (d >= 2 ? kTbBytes : 0);
    hipError_t err = hipSuccess;
    // pick_shape gives the down projection (kScatter, kPartial) a ring of at most 4 k-steps
    constexpr int kMaxDepth = gate_up(EPI) ? 8 : 4;
#define MOE_STREAM_CASE(DEPTH)                                                                                 \
    case DEPTH: {                                                                                              \
        if constexpr (DEPTH > kMaxDepth) return hipErrorInvalidValue;                                           \
        else {                                                                                                 \
        const void* fn = p.deal_active ? reinterpret_cast<const void*>(&ffn_stream_kernel<DEPTH, EPI, true>)    \
                                       : reinterpret_cast<const void*>(&ffn_stream_kernel<DEPTH, EPI, false>);  \
        err = ensure_lds_limit(fn, kLdsMax);                                                                   \
        if (err != hipSuccess) return err;                                                                     \
        const int slots = resident_workgroups(fn, kThreads, lds);                                              \
        const int upw = slots > 0 ? (units + slots - 1) / slots : 1;                                          \
        if (p.deal_active)                                                                                     \
            ffn_stream_kernel<DEPTH, EPI, true><<<(units + upw - 1) / upw, kThreads, lds, stream>>>(p, upw);   \
        else                                                                                                   \
            ffn_stream_kernel<DEPTH, EPI, false><<<(units + upw - 1) / upw, kThreads, lds, stream>>>(p, upw);  \
        break;                                                                                                 \
        }                                                                                                      \
    }
    switch (d) {
        MOE_STREAM_CASE(8)
        MOE_STREAM_CASE(4)
        MOE_STREAM_CASE(2)
        MOE_STREAM_CASE(1)
        default: return hipErrorInvalidValue;
    }
#undef MOE_STREAM_CASE
    err = hipGetLastError();
    return err;
}

// K columns per LDS stage of the wide kernel for a K-range kc: the largest multiple of the ring's batch
// (64 * depth / 2 columns) dividing kc whose `rows` rows fit the LDS beside the re-layout buffers; 0 if none.
int wide_chunk(int kc, int rows, int depth) {
    const int step = 64 * (depth / 2);
    const int max_cols = (kLdsMax - kTbBytes) / (rows * 2) - 8;
    for (int kch = max_cols / step * step; kch >= step; kch -= step)
        if (kc % kch == 0) return kch;
    return 0;
}

template <int EPI, bool LOW>
const void* wide_kernel_fn() {
    return reinterpret_cast<const void*>(&ffn_stream_wide_kernel<EPI, LOW>);
}

// LOW: passes with at most kWideRowsLow rows left run the deeper ring (p.kchunk a multiple of its batch).
template <int EPI, bool LOW>
hipError_t launch_stream_wide(const StreamArgs& p, int units, hipStream_t stream) {
    const size_t lds = static_cast<size_t>(kWideRows) * (p.kchunk + 8) * sizeof(uint16_t) + kTbBytes;
    const void* fn = wide_kernel_fn<EPI, LOW>();
    hipError_t err = ensure_lds_limit(fn, kLdsMax);
    if (err != hipSuccess) return err;
    const int slots = resident_workgroups(fn, kThreads, static_cast<int>(lds));
    const int upw = slots > 0 ? (units + slots - 1) / slots : 1;
    ffn_stream_wide_kernel<EPI, LOW><<<(units + upw - 1) / upw, kThreads, lds, stream>>>(p, upw);
    return hipGetLastError();
}

// The kernel instantiation launch_stream_epi runs for ring depth d (nullptr for none).
template <int EPI, bool DEAL>
const void* stream_kernel_fn(int d) {
    switch (d) {
        case 8:
            if constexpr (gate_up(EPI)) return reinterpret_cast<const void*>(&ffn_stream_kernel<8, EPI, DEAL>);
            else return nullptr;
        case 4: return reinterpret_cast<const void*>(&ffn_stream_kernel<4, EPI, DEAL>);
        case 2: return reinterpret_cast<const void*>(&ffn_stream_kernel<2, EPI, DEAL>);
        case 1: return reinterpret_cast<const void*>(&ffn_stream_kernel<1, EPI, DEAL>);
        default: return nullptr;
    }
}

}  // namespace

hipError_t prepare_ffn_stream(int H, int I) {
    // the 32-row gate/up kernel of either layout that the call's size may pick: whole H, or H split into K-ranges
    const StreamShape whole = pick_shape(H, false), split = gateup_split_shape(H), dn = pick_shape(I, true);
    // the partial-sum kernels at every ring depth, which the tiny batches' K-ranges (tiny_split) may pick
    for (const int d : {8, 4, 2, 1}) {
        for (const void* fn : {stream_kernel_fn<kGatePartial, true>(d), stream_kernel_fn<kPartial, true>(d)}) {
            if (!fn) continue;
            const hipError_t err = ensure_lds_limit(fn, kLdsMax);
            if (err != hipSuccess) return err;
        }
    }
    // each with units dealt over all experts or over the active ones
    for (const bool deal : {false, true}) {
        const void* gu_fns[2] = {
            whole.kc > 0 ? (deal ? stream_kernel_fn<kSwiGLU, true>(whole.d) : stream_kernel_fn<kSwiGLU, false>(whole.d))
                         : nullptr,
            split.kc > 0 && whole.rows_cap != kMaxRows
                ? (deal ? stream_kernel_fn<kGatePartial, true>(split.d) : stream_kernel_fn<kGatePartial, false>(split.d))
                : nullptr};
        if (!gu_fns[0] && !gu_fns[1]) return hipErrorInvalidValue;
        const void* dn_fn = dn.nsplit > 1
                                ? (deal ? stream_kernel_fn<kPartial, true>(dn.d) : stream_kernel_fn<kPartial, false>(dn.d))
                                : (deal ? stream_kernel_fn<kScatter, true>(dn.d) : stream_kernel_fn<kScatter, false>(dn.d));
        const void* fns[3] = {gu_fns[0], gu_fns[1], dn_fn};
        if (!fns[2]) return hipErrorInvalidValue;
        for (const void* fn : fns) {
            if (!fn) continue;
            const hipError_t err = ensure_lds_limit(fn, kLdsMax);
            if (err != hipSuccess) return err;
        }
    }
    if (stream_wide_supported(H, I)) {
        const void* wide_fns[4] = {
            wide_kernel_fn<kSwiGLU, false>(), wide_kernel_fn<kSwiGLU, true>(),
            dn.nsplit > 1 ? wide_kernel_fn<kPartial, false>() : wide_kernel_fn<kScatter, false>(),
            dn.nsplit > 1 ? wide_kernel_fn<kPartial, true>() : wide_kernel_fn<kScatter, true>()};
        for (const void* fn : wide_fns) {
            const hipError_t err = ensure_lds_limit(fn, kLdsMax);
            if (err != hipSuccess) return err;
        }
    }
    return hipSuccess;
}

int stream_block_threads() { return kThreads; }
int stream_rows_per_pass() { return kMaxRows; }

// One fp32 buffer serves both splits in turn: gate/up's sums are reduced into hidden before the down projection
// writes its own. The wide gate/up kernel never splits H.
size_t stream_partial_bytes(int T, int H, int E, int K, int I, bool wide, bool gateup_split) {
    const StreamShape gu = stream_gateup_shape(T, H, E, K, I, wide, gateup_split);
    const StreamShape dn = stream_down_shape(T, H, E, K, I, wide);
    const size_t rows = static_cast<size_t>(T) * K;
    const size_t g = gu.nsplit > 1 ? static_cast<size_t>(gu.nsplit) * rows * 2 * I * sizeof(float) : 0;
    const size_t d = dn.nsplit > 1 ? static_cast<size_t>(dn.nsplit) * rows * H * sizeof(float) : 0;
    return g > d ? g : d;
}

bool stream_supported(int H, int I, bool gateup_split) {
    const bool gu = pick_shape(H, false).kc > 0 || (gateup_split && gateup_split_shape(H).kc > 0);
    return gu && pick_shape(I, true).kc > 0;
}

// Whether the shape can run the wide kernels (both GEMMs' rings and K-ranges allow a chunked stage).
bool stream_wide_supported(int H, int I) {
    const StreamShape gu = gateup_wide_shape(H), dn = pick_shape(I, true);
    return gu.kc > 0 && dn.kc > 0 && wide_chunk(gu.kc, kWideRows, kWideDepth) > 0 &&
           wide_chunk(dn.kc, kWideRows, kWideDepth) > 0;
}
// Whether the wide kernels run their short passes with the deeper ring: up to kWideLowMaxRows rows per expert on
// average, where both GEMMs' K-ranges allow a chunk of 128 rows that is a multiple of that ring's batch.
bool stream_wide_low(int64_t T, int H, int64_t E, int64_t K, int I) {
    const StreamShape gu = gateup_wide_shape(H), dn = pick_shape(I, true);
    return T * K <= kWideLowMaxRows * E && wide_chunk(gu.kc, kWideRows, kWideDepthLow) > 0 &&
           wide_chunk(dn.kc, kWideRows, kWideDepthLow) > 0;
}

// The 32-row kernels stream an expert's weights once per 32 rows, so a single expert above 32 rows doubles the time
// of its units, and those end the launch. The wide kernels therefore run from the average m at which the expected
// largest of E counts of a uniform routing, about m + sqrt(2 ln E * m), passes 32 rows (m ~ 22 at E = 8, 21 at 16,
// 19 at 64, 18 at 256), and from kWideMinRows whatever E. The FFN (32-row / wide kernels, us, two boxes):
//   H = 2048, E = 16, K = 2, I = 8192:   22 rows 267.9 / 293.3, 24 rows 270.7 / 289.9, 26 rows 406.3 / 298.5
//   H = 2048, E = 64, K = 6, I = 1408:   18 rows 189.8 / 220.1, 19.5 rows 281.8 / 223.6, 24 rows 291.2 / 231.3
//   H = 4096, E = 8,  K = 2, I = 14336:  24 rows 521.4 / 500.9, 28 rows 776.8 / 550.4
//   H = 4096, E = 128, K = 8, I = 1536:  20 rows 1290.8 / 827.2
//   H = 7168, E = 256, K = 8, I = 2048:  18 rows 4212.8 / 3637.5, 20 rows 6342.1 / 3714.7
// Skewed routing reaches the second pass at lower averages still; below it the wide kernels cost up to ~10 % more.
// Where 32 rows of H do not fit the LDS (H above 2272) the 32-row gate/up splits H into K-ranges or runs 16-row
// passes, and given enough units to fill the CUs the wide kernels (which stage H in chunks) are faster from fewer
// rows: from 16 rows per expert where 16 rows of H fit (H up to 4568), from 4 where none do (32-row / wide, us):
//   H = 7168, E = 256, K = 8, I = 2048:  4 rows 3520.5 / 3261.1, 8 rows 3791.1 / 3460.3, 16 rows 4101.7 / 3628.6
//   H = 4096, E = 128, K = 8, I = 1536:  8 rows 740.7 / 750.5,  12 rows 843.5 / 782.3, 16 rows 855.9 / 797.1
//   H = 4096, E = 8,   K = 2, I = 14336: 12 rows 486.4 / 501.1, 16 rows 499.7 / 486.6
// With fewer units (H = 5120, E = 16, I = 1536: 192 units of 128 columns for 256 CUs) the 32-row kernels stay
// ahead: 4 / 8 / 16 rows 119.5 / 136.3 / 146.5 against 132.1 / 143.3 / 156.9 us.
constexpr int64_t kWideManyUnits = 512;
int64_t wide_min_rows(int H, int64_t E, int I) {
    const StreamShape whole = pick_shape(H, false);
    if (E * ((I + 127) / 128) < kWideManyUnits || (whole.kc > 0 && whole.rows_cap == kMaxRows)) return kWideMinRows;
    return whole.kc > 0 ? 16 : 4;
}
bool stream_wide(int64_t T, int64_t H, int64_t E, int64_t K, int64_t I) {
    const double m = static_cast<double>(T * K) / static_cast<double>(E);
    const bool past = T * K >= wide_min_rows(static_cast<int>(H), E, static_cast<int>(I)) * E ||
                      m + std::sqrt(2.0 * std::log(static_cast<double>(E)) * m) > kMaxRows;
    return past && stream_wide_supported(static_cast<int>(H), static_cast<int>(I));
}

int stream_gateup_grid(int T, int H, int E, int K, int I, bool wide, bool gateup_split) {
    return E * ((I + kWaves * 16 - 1) / (kWaves * 16)) * stream_gateup_shape(T, H, E, K, I, wide, gateup_split).nsplit;
}

int stream_down_grid(int T, int H, int E, int K, int I, bool wide) {
    return E * ((H + kWaves * 32 - 1) / (kWaves * 32)) * stream_down_shape(T, H, E, K, I, wide).nsplit;
}

hipError_t launch_ffn_stream(const uint16_t* x, const int32_t* expert_ids, const uint16_t* expert_weights,
                             uint16_t* expert_out, const FfnWorkspace& ws, int T, int H, int E, int K, int I,
                             hipStream_t stream, const uint16_t* weights, uint16_t* y, bool gateup_split) {
    StreamArgs p{};
    p.sorted_slot = ws.sorted_slot;
    p.ids = expert_ids;
    p.S = T * K;
    p.deal_active = T * K <= E;
    p.offsets_out = ws.offsets;
    p.sorted_out = ws.sorted_slot;
    p.slot_row_out = ws.slot_row;
    p.expert_out = expert_out;
    p.offsets = ws.offsets;
    p.w = expert_weights;
    p.E = E;
    p.K = K;
    p.H = H;
    p.I = I;
    p.total_rows = T * K;
    // gate/up + SwiGLU: activations = gathered x rows, tiles = W_gate and W_up rows, out = hidden (or, with H split,
    // fp32 partial sums reduced into hidden)
    // experts with more than ~32 rows on average take the wide kernels (up to 128 rows per pass)
    const bool wide = stream_wide(T, H, E, K, I);
    const bool low = wide && stream_wide_low(T, H, E, K, I);
    const StreamShape gu = stream_gateup_shape(T, H, E, K, I, wide, gateup_split);
    p.act = x;
    p.out = ws.hidden;
    p.partial = ws.partial;
    p.kdim = H;
    p.ndim = I;
    p.kc = gu.kc;
    p.rows_cap = gu.rows_cap;
    p.nsplit = gu.nsplit;
    p.w_off = 0;
    p.w1_off = static_cast<size_t>(I) * H;
    p.gather = 1;
    const StreamShape dn = stream_down_shape(T, H, E, K, I, wide);
    hipError_t err;
    {
        TraceScope trace("moe_ffn_gateup_swiglu", stream);
        const int units = stream_gateup_grid(T, H, E, K, I, wide, gateup_split);
        if (wide && low) {
            p.kchunk = wide_chunk(gu.kc, kWideRows, kWideDepthLow);
            err = launch_stream_wide<kSwiGLU, true>(p, units, stream);
        } else if (wide) {
            p.kchunk = wide_chunk(gu.kc, kWideRows, kWideDepth);
            err = launch_stream_wide<kSwiGLU, false>(p, units, stream);
        } else {
            err = gu.nsplit > 1 ? launch_stream_epi<kGatePartial>(p, gu.d, units, stream)
                                : launch_stream_epi<kSwiGLU>(p, gu.d, units, stream);
        }
    }
    if (err != hipSuccess) return err;
    if (gu.nsplit > 1) {
        TraceScope trace("moe_ffn_gateup_reduce", stream);
        const int64_t work = static_cast<int64_t>(T) * K * (I / 8);
        gateup_reduce_kernel<<<static_cast<int>((work + 255) / 256), 256, 0, stream>>>(ws.partial, ws.offsets, E, T * K,
                                                                                        I, gu.nsplit, ws.hidden);
        err = hipGetLastError();
        if (err != hipSuccess) return err;
    }
    // down: activations = hidden rows, tiles = W_down rows n0..n0+15 and n0+16..n0+31
    p.act = ws.hidden;
    p.out = expert_out;
    p.partial = ws.partial;
    p.kdim = I;
    p.ndim = H;
    p.kc = dn.kc;
    p.rows_cap = dn.rows_cap;
    p.nsplit = dn.nsplit;
    p.w_off = 2 * static_cast<size_t>(I) * H;
    p.w1_off = static_cast<size_t>(16) * I;
    p.gather = 0;
    {
        TraceScope trace("moe_ffn_down", stream);
        if (wide && low) {
            p.kchunk = wide_chunk(dn.kc, kWideRows, kWideDepthLow);
            err = dn.nsplit > 1 ? launch_stream_wide<kPartial, true>(p, stream_down_grid(T, H, E, K, I, wide), stream)
                                : launch_stream_wide<kScatter, true>(p, stream_down_grid(T, H, E, K, I, wide), stream);
        } else if (wide) {
            p.kchunk = wide_chunk(dn.kc, kWideRows, kWideDepth);
            err = dn.nsplit > 1 ? launch_stream_wide<kPartial, false>(p, stream_down_grid(T, H, E, K, I, wide), stream)
                                : launch_stream_wide<kScatter, false>(p, stream_down_grid(T, H, E, K, I, wide), stream);
        } else {
            err = dn.nsplit > 1 ? launch_stream_epi<kPartial>(p, dn.d, stream_down_grid(T, H, E, K, I, wide), stream)
                                : launch_stream_epi<kScatter>(p, dn.d, stream_down_grid(T, H, E, K, I, wide), stream);
        }
    }
    if (err != hipSuccess) return err;
    if (dn.nsplit <= 1) return y ? launch_combine(expert_out, weights, y, T, H, K, stream) : hipSuccess;
    if (y) {
        TraceScope trace("moe_ffn_down_reduce_combine", stream);
        const int64_t work = static_cast<int64_t>(T) * (H / 8);
        reduce_combine_kernel<<<static_cast<int>((work + 255) / 256), 256, 0, stream>>>(
            ws.partial, ws.slot_row, expert_ids, weights, E, T, K, H, dn.nsplit, expert_out, y);
    } else {
        TraceScope trace("moe_ffn_down_reduce", stream);
        const int64_t work = static_cast<int64_t>(T) * K * (H / 8);
        down_reduce_kernel<<<static_cast<int>((work + 255) / 256), 256, 0, stream>>>(
            ws.partial, ws.sorted_slot, ws.offsets, E, T * K, H, dn.nsplit, expert_out);
    }
    return hipGetLastError();
}

}  // namespace moe
