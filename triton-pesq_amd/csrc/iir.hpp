// Chunked parallel scan of a bank of parallel second order sections, fp64 state.
//
// A filter is realised in parallel form, y = c0 x + sum_k y_k, where section k
// is a direct form II transposed biquad with b2 = 0 (the form partial
// fractions give; the table packing folds any b2 into the direct term)
//     y_k  = b0 x + z1
//     z1'  = b1 x - a1 y_k + z2
//     z2'  = - a2 y_k
// i.e. the state z = (z1, z2) evolves as z' = A_k z + beta_k x with
// A_k = [[-a1, 1], [-a2, 0]].  Because every A_k is 2x2 and the sections are
// independent, the chunk transfer matrices are block diagonal (4 numbers per
// section) and the scan combine costs 4 FMAs per section.
//
// Geometry.  A lane runs the recursion of all sections over a chunk of kChunk
// consecutive samples (the sections are independent chains, so the lane has
// that much instruction level parallelism); a workgroup is one wavefront and
// covers one block of kBlockSpan = 64 kChunk samples of one row.  Nothing is
// shared between wavefronts, so the kernels have no LDS and no barriers.
//   aggregate: zero state run per chunk, in-wave Kogge-Stone scan; the block's
//              end state per section (given a zero state before the block) is
//              written to `aggr`, laid out [row][section][block][2], and every
//              lane's start state given a zero block start state to `lanes`,
//              laid out [row][block][section][lane][2];
//   prefix:    per (row, section) an exclusive scan of the block aggregates,
//              written over them (aggr[b] becomes the state at the start of
//              block b), one wavefront per sequence; small grids of short rows
//              skip it and the output pass reduces the aggregates before its
//              block instead (block_start_*);
//   output:    lane start state = lanes[lane] + A^(kChunk lane) aggr[block];
//              run from it; per sample y = c0 x + y_0 + y_1 + ... in this order.
// The time axis can be reversed (adjoint filter) by the Mode policy.
//
// Two filters (A and B) can be scanned in the same pass on different inputs;
// the pipeline uses this to run the level-alignment band pass and the
// pre-emphasis filter together.
#pragma once

#include <type_traits>

#include "common.hpp"

namespace pesq {

#ifndef PESQ_CHUNK
#define PESQ_CHUNK 16
#endif
constexpr int kChunk = PESQ_CHUNK;                         // samples per lane
// Lane states: for grids of up to kLaneStateWaves wavefronts (latency bound)
// the aggregate pass stores every lane's in-block start state and the output
// pass reads it; larger grids (bandwidth bound) skip that traffic and the
// output pass repeats the zero state run and the in-wave scan.  Both compute
// the same states up to float64 rounding.
// (8192: grids of up to 7504 wavefronts, such as 8 rows of 60 s, gained 1.5 -
// 4 us from the stored states; 16128, 256 rows of 4 s, was 6 us faster
// recomputing)
constexpr int64_t kLaneStateWaves = 8192;
constexpr int kSpan = kWave * kChunk;                      // samples per block
constexpr int64_t kBlockSpan = kSpan;
#ifndef PESQ_SPLIT_WAVES
#define PESQ_SPLIT_WAVES 3
#endif
// wavefronts per block of the split aggregate pass (each on its own sections)
constexpr int kSplitWaves = PESQ_SPLIT_WAVES;
#ifndef PESQ_SPLIT_OUTPUT
#define PESQ_SPLIT_OUTPUT 1
#endif
// the output pass that warms filter B up (kWarmB) by kOutputWaves wavefronts
// per block, filter A's sections on one, filter B's warm-up and recursion on
// the other (iir_output_split_kernel)
constexpr bool kSplitOutput = PESQ_SPLIT_OUTPUT != 0;
#ifndef PESQ_OUTPUT_WAVES
#define PESQ_OUTPUT_WAVES 2
#endif
constexpr int kOutputWaves = PESQ_OUTPUT_WAVES;
constexpr int kMaxSections = PESQ_IIR_MAX_SECTIONS;
// power levels: A^(kChunk 2^j); j = 0..5 in-wave, 6 = one block, 6..11 the
// block level scan over 64 blocks
constexpr int kLevelBlock = 6;
constexpr int kLevels = 14;
static_assert(kSpan == kChunk << kLevelBlock, "a block is 2^6 chunks");

struct IirTable {
    int32_t na, nb;      // sections of filter A, then of filter B
    double c0a, c0b;     // direct feed through of A and B
    // b2 = 0 in a parallel form table (folded by the packing); kept in the
    // per section tables of a cascade
    double b0[kMaxSections], b1[kMaxSections], b2[kMaxSections];
    double a1[kMaxSections], a2[kMaxSections];
    double pw[kLevels][kMaxSections][4];     // A_k^(kChunk 2^j), row major 2x2
    double lane_pw[kMaxSections][kWave][4];  // A_k^(kChunk lane), lane start powers
    // A_k^(kChunk - 1 - i) beta_k: the weight of the chunk's sample i in the
    // section's state after the chunk, from a zero state (beta_k: the state
    // increment per unit input, (b1 - a1 b0, b2 - a2 b0))
    double fir[kMaxSections][kChunk][2];
    // M^(2 i), M = A_k^kSpan the block transfer: the weight of the block pair
    // (M e_j + e_j+1) 2 i + 2 blocks before a block (block_start_reduce)
    double blk_pw2[kWave][kMaxSections][4];
};

// How an output wavefront obtains its block's start state (the kPrefix
// argument of iir_output_kernel):
//   kStoredStarts  the prefix kernel has replaced the block aggregates by
//                  the block start states (large grids of general filters);
//   kFusedSums     the exact prefix sum over all earlier blocks' aggregates,
//                  formed by the wavefront itself (block_start_load,
//                  block_start_reduce): small grids (those that keep lane
//                  states) of rows of up to kFusedPrefixBlocks blocks;
//   kWindowStarts  the aggregates of the kWarmBlocks blocks before it only
//                  (block_window_load): filters whose state decays below
//                  kWindowDecay over that span (the pipeline's), grids that
//                  keep lane states.  Where the output pass recomputes the
//                  lane states, the window's uniform values would join the
//                  recomputation's coefficients in scalar registers, which
//                  then spill into vector lanes: the prefix pass costs less.
constexpr int kStoredStarts = 0;
constexpr int kFusedSums = 1;
constexpr int kWindowStarts = 2;
#ifndef PESQ_FUSED_PREFIX_BLOCKS
#define PESQ_FUSED_PREFIX_BLOCKS 128
#endif
constexpr int kFusedPrefixBlocks = PESQ_FUSED_PREFIX_BLOCKS;
static_assert(kFusedPrefixBlocks <= 2 * kWave, "two blocks per lane");

// Windowed block starts.  A block's start state differs from the end state
// of the kWarmBlocks blocks before it, run from a zero state, by
// A^(kWarmBlocks kSpan) applied to the state there, i.e. by at most twice
// kWindowDecay of the state's largest component when every entry of that
// matrix power is below kWindowDecay (checked for every section where the
// pipeline's table is packed).  For the PESQ filters (pole radii up to 0.968
// for the level alignment filter, 0.973 for the pre-emphasis filter) the
// largest entry of A^2048 is 3e-24, far below the float64 rounding of the
// recursion.  So an output wavefront takes its block start state from the
// aggregates of the two blocks before it (kWindowStarts), with no prefix
// pass, and the backward's output pass forms filter B's block start states
// from that filter's inputs in those blocks (kWarmB), with no aggregate pass
// for it.
constexpr int kWarmBlocks = 2;
constexpr double kWindowDecay = 1e-20;

// Launch plan of a scan over `rows` rows of nblk blocks (one wavefront each):
// whether the aggregate pass stores the lane states, and whether the output
// pass derives the block start states itself (no prefix launch).  The
// workspace sizing and the launches both read it.
struct ScanPlan {
    bool lane_states;
    bool fused_prefix;
};
__host__ __device__ __forceinline__ ScanPlan scan_plan(int64_t rows, int64_t nblk) {
    const bool lanes = rows * nblk <= kLaneStateWaves;
    return {lanes, lanes && nblk <= kFusedPrefixBlocks};
}

// Scan workspace of `rows` rows of nblk blocks and `ns` sections: the block
// aggregates [row][section][block][2], then, when the plan stores them, the
// lane states [row][block][section][lane][2].
__host__ __device__ __forceinline__ int64_t scan_aggr_doubles(int64_t rows, int64_t nblk,
                                                              int ns = kMaxSections) {
    return rows * nblk * ns * 2;
}
__host__ __device__ __forceinline__ int64_t scan_workspace_doubles(int64_t rows, int64_t nblk,
                                                                   int ns = kMaxSections) {
    const int64_t lanes = scan_plan(rows, nblk).lane_states ? kWave : 0;
    return scan_aggr_doubles(rows, nblk, ns) * (1 + lanes);
}

// --------------------------------------------------------------------------
// per lane state of a bank of NS sections starting at section S0
// --------------------------------------------------------------------------

template <int NS>
struct Bank {
    double u[NS > 0 ? NS : 1], v[NS > 0 ? NS : 1];  // z1, z2 per section

    __device__ __forceinline__ void zero() {
#pragma unroll
        for (int k = 0; k < NS; ++k) u[k] = v[k] = 0.0;
    }
};

// Coefficients of NS sections starting at section S0.  With kB2 the sections
// are full biquads (z2' = b2 x - a2 y_k, the cascade passes); without it b2 is
// 0 (the parallel form, whose table packing folds b2 into the direct term).
template <int S0, int NS, bool kB2 = false>
struct Coeffs {
    double b0[NS > 0 ? NS : 1], b1[NS > 0 ? NS : 1], b2[NS > 0 ? NS : 1];
    double a1[NS > 0 ? NS : 1], a2[NS > 0 ? NS : 1];
    double c0;

    __device__ __forceinline__ void load(const IirTable &t, double direct) {
#pragma unroll
        for (int k = 0; k < NS; ++k) {
            b0[k] = t.b0[S0 + k];
            b1[k] = t.b1[S0 + k];
            b2[k] = kB2 ? t.b2[S0 + k] : 0.0;
            a1[k] = t.a1[S0 + k];
            a2[k] = t.a2[S0 + k];
        }
        c0 = direct;
    }

    // one time step: consumes x, advances the state, returns c0 x + sum_k y_k
    __device__ __forceinline__ double step(Bank<NS> &s, double x) const {
        double y = c0 * x;
#pragma unroll
        for (int k = 0; k < NS; ++k) {
            const double yk = fma(b0[k], x, s.u[k]);
            s.u[k] = fma(-a1[k], yk, fma(b1[k], x, s.v[k]));
            s.v[k] = kB2 ? fma(b2[k], x, -a2[k] * yk) : -a2[k] * yk;
            y += yk;
        }
        return y;
    }
    // the same step, each section's output kept apart (y[k] = y_k)
    __device__ __forceinline__ void step_parts(Bank<NS> &s, double x,
                                               double (&y)[NS > 0 ? NS : 1]) const {
#pragma unroll
        for (int k = 0; k < NS; ++k) {
            const double yk = fma(b0[k], x, s.u[k]);
            s.u[k] = fma(-a1[k], yk, fma(b1[k], x, s.v[k]));
            s.v[k] = kB2 ? fma(b2[k], x, -a2[k] * yk) : -a2[k] * yk;
            y[k] = yk;
        }
    }
};

// z <- P z + add, P = A_k^(kChunk 2^level) per section
template <int S0, int NS>
__device__ __forceinline__ void apply_power(const IirTable &t, int level, Bank<NS> &z,
                                            const Bank<NS> &add) {
#pragma unroll
    for (int k = 0; k < NS; ++k) {
        const double *p = t.pw[level][S0 + k];
        const double u = z.u[k], v = z.v[k];
        z.u[k] = fma(p[0], u, fma(p[1], v, add.u[k]));
        z.v[k] = fma(p[2], u, fma(p[3], v, add.v[k]));
    }
}

// Inclusive Kogge-Stone scan over the 64 lanes of a wavefront.  Element c is
// a state contribution at the end of chunk c; after the scan lane c holds
// sum_{i <= c} A^((c - i) stride) e_i with stride = kChunk 2^level0.
template <int S0, int NS>
__device__ __forceinline__ void scan_wave(const IirTable &t, int level0, Bank<NS> &z, int lane) {
#pragma unroll
    for (int j = 0; j < 6; ++j) {
        const int d = 1 << j;
        Bank<NS> o;
#pragma unroll
        for (int k = 0; k < NS; ++k) {
            o.u[k] = shfl_up(z.u[k], d);
            o.v[k] = shfl_up(z.v[k], d);
        }
        if (lane >= d) {
            apply_power<S0, NS>(t, level0 + j, o, z);  // o <- P o + z
            z = o;
        }
    }
}

// The same inclusive scan with DPP lane moves instead of LDS crossbar
// shuffles (GFX9 DPP, 64-bit values as two 32-bit moves): Kogge-Stone over
// the 16 lanes of each row (row_shr 1, 2, 4, 8; lanes shifted in from
// outside the row read 0), then the last lane of row 0 (of row 2) is carried
// into row 1 (row 3) with row_bcast:15, and the last lane of row 1 into rows 2
// and 3 with row_bcast:31, each lane scaling the carry by A^(kChunk m), m its
// distance in chunks from the carried lane (lane_pw).  For level0 = 0 only.
template <int kCtrl, int kRowMask>
__device__ __forceinline__ double dpp_move(double v) {
    const int lo = __builtin_amdgcn_update_dpp(0, __double2loint(v), kCtrl, kRowMask, 0xF, true);
    const int hi = __builtin_amdgcn_update_dpp(0, __double2hiint(v), kCtrl, kRowMask, 0xF, true);
    return __hiloint2double(hi, lo);
}

template <int kCtrl, int kRowMask, int S0, int NS>
__device__ __forceinline__ void dpp_level(const double *const (&pw)[NS > 0 ? NS : 1], Bank<NS> &z) {
#pragma unroll
    for (int k = 0; k < NS; ++k) {
        const double ou = dpp_move<kCtrl, kRowMask>(z.u[k]);
        const double ov = dpp_move<kCtrl, kRowMask>(z.v[k]);
        const double *p = pw[k];
        z.u[k] = fma(p[0], ou, fma(p[1], ov, z.u[k]));
        z.v[k] = fma(p[2], ou, fma(p[3], ov, z.v[k]));
    }
}

template <int S0, int NS, class Powers>
__device__ __forceinline__ void scan_wave_dpp(const Powers &t, Bank<NS> &z, int lane) {
    const double *pw[NS > 0 ? NS : 1];
#pragma unroll
    for (int k = 0; k < NS; ++k) pw[k] = t.pw[0][S0 + k];
    dpp_level<0x111, 0xF, S0, NS>(pw, z);  // row_shr:1
#pragma unroll
    for (int k = 0; k < NS; ++k) pw[k] = t.pw[1][S0 + k];
    dpp_level<0x112, 0xF, S0, NS>(pw, z);  // row_shr:2
#pragma unroll
    for (int k = 0; k < NS; ++k) pw[k] = t.pw[2][S0 + k];
    dpp_level<0x114, 0xF, S0, NS>(pw, z);  // row_shr:4
#pragma unroll
    for (int k = 0; k < NS; ++k) pw[k] = t.pw[3][S0 + k];
    dpp_level<0x118, 0xF, S0, NS>(pw, z);  // row_shr:8
    // rows 1 and 3: + A^(kChunk ((lane & 15) + 1)) (lane 15 of rows 0 and 2)
#pragma unroll
    for (int k = 0; k < NS; ++k) pw[k] = t.lane_pw[S0 + k][(lane & 15) + 1];
    dpp_level<0x142, 0xA, S0, NS>(pw, z);  // row_bcast:15
    // rows 2 and 3: + A^(kChunk (lane - 31)) (lane 31)
#pragma unroll
    for (int k = 0; k < NS; ++k) pw[k] = t.lane_pw[S0 + k][lane >= 32 ? lane - 31 : 0];
    dpp_level<0x143, 0xC, S0, NS>(pw, z);  // row_bcast:31
}

// Start state of block `blk` of a row from the zero start end states e_j of
// the blocks before it (row_aggr, laid out [section][block][2]):
//     p = sum_{j < blk} M^(blk - 1 - j) e_j,  M = A^kSpan per section.
// Lane i holds blocks j0 = blk - 128 + 2 i and j0 + 1 (0 before the row
// start), combines them as M e_j0 + e_j0+1 and carries the pair to the block
// start with M^(2 (63 - i)) (blk_pw2); the 64 lanes' terms are then summed in
// LDS (wave_sums_lds, `red`) and every lane reads the sums back.  The loads are
// issued first so that they overlap the kernel's other loads.
template <int NS, int NL = NS>
__device__ __forceinline__ void block_start_load(const double *row_aggr, int nblk, int blk,
                                                 int lane, Bank<NS> &e0, Bank<NS> &e1) {
    // sections NL .. NS - 1 (none by default) take no aggregates: zero
#pragma unroll
    for (int k = NL; k < NS; ++k) e0.u[k] = e0.v[k] = e1.u[k] = e1.v[k] = 0.0;
    const int j0 = blk - 2 * kWave + 2 * lane;
    const int c0 = j0 >= 0 ? j0 : 0, c1 = j0 + 1 >= 0 ? j0 + 1 : 0;
#pragma unroll
    for (int k = 0; k < NL; ++k) {
        const double *sec = row_aggr + int64_t(k) * nblk * 2;
        const double2 a = *reinterpret_cast<const double2 *>(sec + 2 * c0);
        const double2 b = *reinterpret_cast<const double2 *>(sec + 2 * c1);
        e0.u[k] = j0 >= 0 ? a.x : 0.0;
        e0.v[k] = j0 >= 0 ? a.y : 0.0;
        e1.u[k] = j0 + 1 >= 0 ? b.x : 0.0;
        e1.v[k] = j0 + 1 >= 0 ? b.y : 0.0;
    }
}

// Start state of block `blk` of a row from the zero start end states of the
// kWarmBlocks = 2 blocks before it (windowed block starts, above):
//     p = e_(blk-1) + M e_(blk-2),  M = A^kSpan per section.
// The addresses are uniform over the wavefront.  e0 receives e_(blk-2), e1
// e_(blk-1) (0 before the row start; sections NL .. NS - 1 take none);
// block_window_start then leaves p in e0.
template <int NS, int NL = NS>
__device__ __forceinline__ void block_window_load(const double *row_aggr, int nblk, int blk,
                                                  Bank<NS> &e0, Bank<NS> &e1) {
    static_assert(kWarmBlocks == 2, "a window of two blocks");
#pragma unroll
    for (int k = NL; k < NS; ++k) e0.u[k] = e0.v[k] = e1.u[k] = e1.v[k] = 0.0;
    const int c0 = blk >= 2 ? blk - 2 : 0, c1 = blk >= 1 ? blk - 1 : 0;
#pragma unroll
    for (int k = 0; k < NL; ++k) {
        const double *sec = row_aggr + int64_t(k) * nblk * 2;
        const double2 a = *reinterpret_cast<const double2 *>(sec + 2 * c0);
        const double2 b = *reinterpret_cast<const double2 *>(sec + 2 * c1);
        e0.u[k] = blk >= 2 ? a.x : 0.0;
        e0.v[k] = blk >= 2 ? a.y : 0.0;
        e1.u[k] = blk >= 1 ? b.x : 0.0;
        e1.v[k] = blk >= 1 ? b.y : 0.0;
    }
}
template <int NS, int S0 = 0>
__device__ __forceinline__ void block_window_start(const IirTable &t, Bank<NS> &e0,
                                                   const Bank<NS> &e1) {
#pragma unroll
    for (int k = 0; k < NS; ++k) {
        const double *m = t.pw[kLevelBlock][S0 + k];
        const double u = fma(m[0], e0.u[k], fma(m[1], e0.v[k], e1.u[k]));
        const double v = fma(m[2], e0.u[k], fma(m[3], e0.v[k], e1.v[k]));
        e0.u[k] = u;
        e0.v[k] = v;
    }
}

// Modes whose output pass reads per row constants from memory (Mode::Pre,
// m.prefetch(row, lane, pre) issuing the loads, m.setup(row, sh, lane, pre)
// using them): the output kernel requests them before its raw inputs.
template <class M, class = void>
struct HasPre : std::false_type {};
template <class M>
struct HasPre<M, std::void_t<typename M::Pre>> : std::true_type {};

// the lane's pair power M^(2 (63 - lane)) of every section, loaded with the
// block end states (block_start_load) so that its latency overlaps theirs
template <int NS>
struct PairPowers {
    double2 m[NS > 0 ? NS : 1][2];

    __device__ __forceinline__ void load(const IirTable &t, int lane) {
#pragma unroll
        for (int k = 0; k < NS; ++k) {
            const double2 *q = reinterpret_cast<const double2 *>(t.blk_pw2[kWave - 1 - lane][k]);
            m[k][0] = q[0];
            m[k][1] = q[1];
        }
    }
};

template <int NS>
__device__ __forceinline__ void block_start_reduce(const IirTable &t, const PairPowers<NS> &pp,
                                                   Bank<NS> &z, const Bank<NS> &e1, double *red,
                                                   int lane) {
    double w[2 * NS];
#pragma unroll
    for (int k = 0; k < NS; ++k) {
        const double *m = t.pw[kLevelBlock][k];
        const double u = fma(m[0], z.u[k], fma(m[1], z.v[k], e1.u[k]));
        const double v = fma(m[2], z.u[k], fma(m[3], z.v[k], e1.v[k]));
        const double2 q0 = pp.m[k][0], q1 = pp.m[k][1];
        w[2 * k] = fma(q0.x, u, q0.y * v);
        w[2 * k + 1] = fma(q1.x, u, q1.y * v);
    }
    const double sum = wave_sums_lds(w, red, lane);  // component j in lane 4 j
    if (lane % 4 == 0 && lane / 4 < 2 * NS) red[lane / 4] = sum;
    wave_lds_fence();
#pragma unroll
    for (int k = 0; k < NS; ++k) {
        z.u[k] = red[2 * k];
        z.v[k] = red[2 * k + 1];
    }
    wave_lds_fence();
}

// The states of NA sections of filter A and NB of filter B, which are the
// table's sections kBase .. kBase + NA - 1 and kBase + NA .. kBase + NA + NB - 1
// (kBase 0: all sections of both filters; a pass may also run a subset).
template <int NA, int NB, int kBase = 0>
struct BankPair {
    Bank<NA> a;
    Bank<NB> b;

    __device__ __forceinline__ void zero() {
        a.zero();
        b.zero();
    }
    __device__ __forceinline__ void scan(const IirTable &t, int level0, int lane) {
        if constexpr (NA > 0) scan_wave<kBase, NA>(t, level0, a, lane);
        if constexpr (NB > 0) scan_wave<kBase + NA, NB>(t, level0, b, lane);
    }
    // the in-wave chunk scan (level0 = 0) with DPP moves
    template <class Powers>
    __device__ __forceinline__ void scan_chunks(const Powers &t, int lane) {
        if constexpr (NA > 0) scan_wave_dpp<kBase, NA>(t, a, lane);
        if constexpr (NB > 0) scan_wave_dpp<kBase + NA, NB>(t, b, lane);
    }
    __device__ __forceinline__ void power(const IirTable &t, int level, const BankPair &add) {
        if constexpr (NA > 0) apply_power<kBase, NA>(t, level, a, add.a);
        if constexpr (NB > 0) apply_power<kBase + NA, NB>(t, level, b, add.b);
    }
    // section k (0 .. NA + NB - 1) as (u, v) references
    __device__ __forceinline__ double &u(int k) { return k < NA ? a.u[k] : b.u[k - NA]; }
    __device__ __forceinline__ double &v(int k) { return k < NA ? a.v[k] : b.v[k - NA]; }
};

// --------------------------------------------------------------------------
// the kernels, parametrised by a Mode policy:
//   Mode::kInputs                 raw inputs per sample (1 or 2)
//   Mode::kOutputs                outputs per sample (1 or 2)
//   Mode::In, Mode::Out           element types of the raw inputs and the
//                                 outputs in memory (float or double)
//   Mode::kB2                     full biquad sections (b2 read from the table)
//   Mode::kReverse                process the time axis back to front
//   Mode::kAccumulates            the output pass reduces a per block sum
//   Mode::kRamp                   the Mode uses the edge ramp weight w of the
//                                 sample (edge_weight(n, len)); otherwise the
//                                 kernels pass w = 1
//   m.src(row, q)                 row base of raw input q (physical order)
//   m.dst(row, q)                 row base of output q, or null when the row
//                                 does not write that output
//   m.inputs(w, in[], xa, xb)     filter inputs of a sample from its raw inputs
//   m.setup(row, sh, lane)        output pass: per row constants into sh[0..3]
//                                 (wave-uniform values)
//   m.compute(w, ya, yb, acc, sh, out[]) the outputs of a sample from the
//                                 outputs ya, yb of the two filters
//   m.finish(row, blk, total)     block total of the accumulator
// The scan is linear, so it runs in the units of the raw inputs; per row
// constants are applied by compute.
//
// Memory access: a lane reads and writes its kChunk consecutive samples as
// 16-byte vectors when the row's alignment allows it (the whole wavefront
// then covers kSpan contiguous samples per instruction group), else element
// by element; the last chunk of a row is handled element by element.
// --------------------------------------------------------------------------

// physical index of the first sample of a full chunk starting at time j0
template <bool kRev>
__device__ __forceinline__ int64_t chunk_lo(int64_t j0, int64_t len) {
    return kRev ? len - j0 - kChunk : j0;
}

// 16-byte vector moves of float (4 per vector) and double (2 per vector)
__device__ __forceinline__ void load16(const float *p, float *dst) {
    const float4 w = *reinterpret_cast<const float4 *>(p);
    dst[0] = w.x;
    dst[1] = w.y;
    dst[2] = w.z;
    dst[3] = w.w;
}
__device__ __forceinline__ void load16(const double *p, double *dst) {
    const double2 w = *reinterpret_cast<const double2 *>(p);
    dst[0] = w.x;
    dst[1] = w.y;
}
__device__ __forceinline__ void store16(float *p, const float *src) {
    *reinterpret_cast<float4 *>(p) = make_float4(src[0], src[1], src[2], src[3]);
}
__device__ __forceinline__ void store16(double *p, const double *src) {
    *reinterpret_cast<double2 *>(p) = make_double2(src[0], src[1]);
}

// One path for all inputs (16-byte vectors when every input's chunk is full
// and aligned, else elements), so that the loads of all inputs are issued
// before the first wait for one of them.
template <class Mode>
__device__ __forceinline__ void load_chunk(const Mode &m, int row, int64_t j0, int64_t len,
                                           typename Mode::In (&in)[kChunk][Mode::kInputs]) {
    using T = typename Mode::In;
    constexpr int kVec = 16 / sizeof(T);
    const bool full = j0 + kChunk <= len;
    const int64_t lo = chunk_lo<Mode::kReverse>(j0, len);
    bool vec = full;
#pragma unroll
    for (int q = 0; q < Mode::kInputs; ++q) {
        vec = vec && (reinterpret_cast<uintptr_t>(m.src(row, q) + lo) & 15) == 0;
    }
    if (vec) {
        T buf[Mode::kInputs][kChunk];
#pragma unroll
        for (int q = 0; q < Mode::kInputs; ++q) {
            const T *base = m.src(row, q);
#pragma unroll
            for (int r = 0; r < kChunk / kVec; ++r) load16(base + lo + kVec * r, buf[q] + kVec * r);
        }
#pragma unroll
        for (int q = 0; q < Mode::kInputs; ++q) {
#pragma unroll
            for (int i = 0; i < kChunk; ++i) in[i][q] = buf[q][Mode::kReverse ? kChunk - 1 - i : i];
        }
    } else {
#pragma unroll
        for (int q = 0; q < Mode::kInputs; ++q) {
            const T *base = m.src(row, q);
#pragma unroll
            for (int i = 0; i < kChunk; ++i) {
                const int64_t j = j0 + i;
                const int64_t jc = j < len ? j : len - 1;
                const T v = base[Mode::kReverse ? len - 1 - jc : jc];
                in[i][q] = j < len ? v : T(0);
            }
        }
    }
}

// out[i] is stored at time index j0 + i
template <typename T>
__device__ __forceinline__ void store_chunk(T *base, const T (&out)[kChunk], bool kRev,
                                            int64_t j0, int64_t len) {
    constexpr int kVec = 16 / sizeof(T);
    const bool full = j0 + kChunk <= len;
    const int64_t lo = kRev ? len - j0 - kChunk : j0;
    if (full && (reinterpret_cast<uintptr_t>(base + lo) & 15) == 0) {
        T e[kChunk];
#pragma unroll
        for (int i = 0; i < kChunk; ++i) e[i] = out[kRev ? kChunk - 1 - i : i];
#pragma unroll
        for (int r = 0; r < kChunk / kVec; ++r) store16(base + lo + kVec * r, e + kVec * r);
    } else {
#pragma unroll
        for (int i = 0; i < kChunk; ++i) {
            const int64_t j = j0 + i;
            if (j < len) base[kRev ? len - 1 - j : j] = out[i];
        }
    }
}

// A chunk is "general" when it reaches within kEdge samples of a row end (or
// past it): only there do the edge ramp weights differ from 1 and time indices
// fall outside the row.  Interior chunks take a path without either check.
__device__ __forceinline__ bool general_chunk(int64_t j0, int64_t len) {
    return j0 < kEdge || j0 + kChunk + kEdge > len;
}

// filter inputs of element i (time index j0 + i) of a chunk
template <bool kGeneral, class Mode>
__device__ __forceinline__ void element_inputs(const Mode &m,
                                               const typename Mode::In (&in)[Mode::kInputs],
                                               int64_t j, int64_t len, double &w, double &xa,
                                               double &xb) {
    w = 1.0;
    if constexpr (kGeneral && Mode::kRamp) {
        if (j < len) w = edge_weight(Mode::kReverse ? len - 1 - j : j, len);
    }
    m.inputs(w, in, xa, xb);
    if constexpr (kGeneral) {
        if (j >= len) xa = xb = 0.0;
    }
}

// state of NS sections from S0 after the chunk, from a zero state, as the
// weighted sums of the chunk's inputs x[0 .. kChunk - 1]: kChunk independent
// fused multiply-adds per state component instead of the recursion's chain
template <int S0, int NS>
__device__ __forceinline__ void chunk_end_state(const IirTable &t, const double (&x)[kChunk],
                                                Bank<NS> &s) {
#pragma unroll
    for (int k = 0; k < NS; ++k) {
        double u = t.fir[S0 + k][0][0] * x[0];
        double v = t.fir[S0 + k][0][1] * x[0];
#pragma unroll
        for (int i = 1; i < kChunk; ++i) {
            u = fma(t.fir[S0 + k][i][0], x[i], u);
            v = fma(t.fir[S0 + k][i][1], x[i], v);
        }
        s.u[k] = u;
        s.v[k] = v;
    }
}

// zero state run over the lane's chunk: the state after it.  With kWeighted,
// interior chunks form it as weighted sums of the inputs (chunk_end_state):
// fewer and independent operations (14 us at BASELINE c5; at c2 the split
// aggregate pass, two sections per wavefront and issue bound, gained 0.6 us,
// where the one-wavefront pass over six sections had lost 1 us to the
// weights' scalar loads).  Chunks at a row end always run the recursion,
// with the ramp weights and bounds of element_inputs.
template <bool kGeneral, bool kWeighted, int NA, int NB, class Mode, int kBase = 0>
__device__ __forceinline__ void zero_run(const Mode &m, const IirTable &t,
                                         const Coeffs<kBase, NA, Mode::kB2> &ca,
                                         const Coeffs<kBase + NA, NB, Mode::kB2> &cb,
                                         const typename Mode::In (&in)[kChunk][Mode::kInputs],
                                         int64_t j0,
                                         int64_t len, BankPair<NA, NB, kBase> &s) {
    if constexpr (kGeneral || !kWeighted) {
#pragma unroll
        for (int i = 0; i < kChunk; ++i) {
            double w, xa, xb;
            element_inputs<kGeneral>(m, in[i], j0 + i, len, w, xa, xb);
            if constexpr (NA > 0) ca.step(s.a, xa);
            if constexpr (NB > 0) cb.step(s.b, xb);
        }
    } else {
        double xa[kChunk], xb[kChunk];
#pragma unroll
        for (int i = 0; i < kChunk; ++i) {
            double w;
            element_inputs<false>(m, in[i], j0 + i, len, w, xa[i], xb[i]);
        }
        if constexpr (NA > 0) chunk_end_state<kBase, NA>(t, xa, s.a);
        if constexpr (NB > 0) chunk_end_state<kBase + NA, NB>(t, xb, s.b);
    }
}

// run from the true start state s, outputs into out[][i]
template <bool kGeneral, int NA, int NB, class Mode>
__device__ __forceinline__ void output_run(const Mode &m, const Coeffs<0, NA, Mode::kB2> &ca,
                                           const Coeffs<NA, NB, Mode::kB2> &cb,
                                           const typename Mode::In (&in)[kChunk][Mode::kInputs],
                                           int64_t j0, int64_t len, const double *sh,
                                           BankPair<NA, NB> &s,
                                           typename Mode::Out (&out)[Mode::kOutputs][kChunk],
                                           double &acc) {
#pragma unroll
    for (int i = 0; i < kChunk; ++i) {
        const int64_t j = j0 + i;
        double w, xa, xb;
        element_inputs<kGeneral>(m, in[i], j, len, w, xa, xb);
        double ya = 0.0, yb = 0.0;
        if constexpr (NA > 0) ya = ca.step(s.a, xa);
        if constexpr (NB > 0) yb = cb.step(s.b, xb);
        typename Mode::Out o[Mode::kOutputs];
        const double before = acc;
        m.compute(w, ya, yb, acc, sh, o);
        if constexpr (kGeneral) {
            if (j >= len) acc = before;  // past the end of the row
        }
#pragma unroll
        for (int q = 0; q < Mode::kOutputs; ++q) {
            out[q][i] = (!kGeneral || j < len) ? o[q] : typename Mode::Out(0);
        }
    }
}

// The block's end state from a zero start state, when no lane state is
// needed: sum over the lanes c of A^(kChunk (63 - c)) e_c, e_c the lane's chunk
// end state from zero (s), instead of the in-wave scan (which also gives every
// lane's start state); component j (section j / 2) is summed in LDS by
// wave_sums_lds and stored by lane 4 j at dst[j / 2 section stride + j % 2]
// (dst: section 0 of this block, sections nblk * 2 doubles apart).
template <int NS, class BP>
__device__ __forceinline__ void block_end_state(const IirTable &t, BP &s, double *dst, int nblk,
                                                int lane) {
    constexpr int kComps = 2 * NS;
    __shared__ double red[wave_sums_lds_doubles<kComps>()];
    double w[kComps];
#pragma unroll
    for (int k = 0; k < NS; ++k) {
        const double *lp = t.lane_pw[k][kWave - 1 - lane];
        const double u = s.u(k), v = s.v(k);
        w[2 * k] = fma(lp[0], u, lp[1] * v);
        w[2 * k + 1] = fma(lp[2], u, lp[3] * v);
    }
    const double sum = wave_sums_lds(w, red, lane);
    const int comp = lane / 4;
    if (lane % 4 == 0 && comp < kComps) dst[int64_t(comp / 2) * nblk * 2 + comp % 2] = sum;
}

// The aggregate pass of one block (row, blk) by one wavefront, lane states
// stored: sections kBase .. kBase + NA + NB - 1 of a workspace laid out for
// kLayout sections (the aggregates [row][section][block][2], the lane states
// [row][block][section][lane][2]).  Every section is an independent
// recursion, so a pass over a subset of the sections writes the same bits for
// them as a pass over all (the pipeline runs the backward's level alignment
// filter on its own, inside an earlier kernel, and the pre-emphasis filter in
// the aggregate launch).
template <int NA, int NB, int kBase, int kLayout, class Mode>
__device__ __forceinline__ void aggregate_block(const Mode &m, const IirTable &t, double *aggr,
                                                double *lanes, int64_t len, int nblk, int row,
                                                int blk, int lane) {
    constexpr int NS = NA + NB;
    static_assert(kBase + NS <= kLayout, "sections inside the layout");
    const int64_t j0 = int64_t(blk) * kSpan + int64_t(lane) * kChunk;
    Coeffs<kBase, NA, Mode::kB2> ca;
    Coeffs<kBase + NA, NB, Mode::kB2> cb;
    ca.load(t, t.c0a);
    cb.load(t, t.c0b);

    typename Mode::In in[kChunk][Mode::kInputs];
    load_chunk(m, row, j0, len, in);

    BankPair<NA, NB, kBase> s;
    s.zero();
    if (general_chunk(j0, len)) {
        zero_run<true, false>(m, t, ca, cb, in, j0, len, s);
    } else {
        zero_run<false, true>(m, t, ca, cb, in, j0, len, s);
    }
    s.scan_chunks(t, lane);
    if (lane == kWave - 1) {
#pragma unroll
        for (int k = 0; k < NS; ++k) {
            double *dst = aggr + ((int64_t(row) * kLayout + kBase + k) * nblk + blk) * 2;
            dst[0] = s.u(k);
            dst[1] = s.v(k);
        }
    }
    // start state of every lane's chunk (the end state of the chunk before it)
    double2 *dst = reinterpret_cast<double2 *>(lanes) +
                   ((int64_t(row) * nblk + blk) * kLayout + kBase) * kWave;
#pragma unroll
    for (int k = 0; k < NS; ++k) {
        // wave_shr:1 (lane 0 reads 0)
        const double u = dpp_move<0x138, 0xF>(s.u(k)), v = dpp_move<0x138, 0xF>(s.v(k));
        dst[k * kWave + lane] = make_double2(u, v);
    }
}

template <int NA, int NB, class Mode, bool kLaneStates, int kBase = 0, int kLayout = NA + NB>
__global__ void __launch_bounds__(kWave)
    iir_aggregate_kernel(Mode m, const IirTable *__restrict__ table, double *__restrict__ aggr,
                         double *__restrict__ lanes, int64_t len, int nblk) {
    const IirTable &t = *table;
    const int row = blockIdx.x / nblk;
    const int blk = blockIdx.x - row * nblk;
    const int lane = threadIdx.x;
    if constexpr (kLaneStates) {
        aggregate_block<NA, NB, kBase, kLayout>(m, t, aggr, lanes, len, nblk, row, blk, lane);
    } else {
        static_assert(kBase == 0 && kLayout == NA + NB, "all sections without lane states");
        constexpr int NS = NA + NB;
        const int64_t j0 = int64_t(blk) * kSpan + int64_t(lane) * kChunk;
        Coeffs<0, NA, Mode::kB2> ca;
        Coeffs<NA, NB, Mode::kB2> cb;
        ca.load(t, t.c0a);
        cb.load(t, t.c0b);
        typename Mode::In in[kChunk][Mode::kInputs];
        load_chunk(m, row, j0, len, in);
        BankPair<NA, NB> s;
        s.zero();
        if (general_chunk(j0, len)) {
            zero_run<true, true>(m, t, ca, cb, in, j0, len, s);
        } else {
            zero_run<false, true>(m, t, ca, cb, in, j0, len, s);
        }
        block_end_state<NS>(t, s, aggr + (int64_t(row) * NS * nblk + blk) * 2, nblk, lane);
    }
}

// The aggregate pass with lane states by kWaves wavefronts per block, each on
// its own sections: wavefront w runs sections [w NS / kWaves, (w + 1) NS /
// kWaves) of the NS = NA + NB (A's sections first, then B's).  The sections
// are independent recursions, so this writes the same bits as
// iir_aggregate_kernel, with 1 / kWaves of the serial work per wavefront (all
// of them read the block's inputs).
template <int NA, int NB, int kWaves, int W, class Mode>
__device__ __forceinline__ void aggregate_split_wave(const Mode &m, const IirTable &t, double *aggr,
                                                     double *lanes, int64_t len, int nblk, int row,
                                                     int blk, int lane, int w) {
    constexpr int NS = NA + NB;
    constexpr int lo = W * NS / kWaves, hi = (W + 1) * NS / kWaves;
    constexpr int na = (hi < NA ? hi : NA) - (lo < NA ? lo : NA);  // A's sections in [lo, hi)
    constexpr int nb = hi - lo - na;
    if (w == W) {
        aggregate_block<na, nb, lo, NS>(m, t, aggr, lanes, len, nblk, row, blk, lane);
    } else if constexpr (W + 1 < kWaves) {
        aggregate_split_wave<NA, NB, kWaves, W + 1>(m, t, aggr, lanes, len, nblk, row, blk, lane,
                                                     w);
    }
}

template <int NA, int NB, int kWaves, class Mode>
__global__ void __launch_bounds__(kWaves * kWave)
    iir_aggregate_split_kernel(Mode m, const IirTable *__restrict__ table,
                               double *__restrict__ aggr, double *__restrict__ lanes, int64_t len,
                               int nblk) {
    static_assert(kWaves >= 2 && kWaves <= NA + NB, "one section per wavefront at least");
    const IirTable &t = *table;
    const int row = blockIdx.x / nblk;
    const int blk = blockIdx.x - row * nblk;
    const int lane = threadIdx.x % kWave;
    aggregate_split_wave<NA, NB, kWaves, 0>(m, t, aggr, lanes, len, nblk, row, blk, lane,
                                            wave_index());
}

// Exclusive scan of the block aggregates, one (row, section) sequence per
// wavefront; aggr[b] is replaced by the state at the start of block b
// (s_{b+1} = M s_b + e_b, M = A^1024 the block transfer, e_b the aggregate).
// Lane l owns the per = ceil(nblk / 64) consecutive blocks l per .. l per +
// per - 1: it runs them from a zero start (its chunk total), a Kogge-Stone
// scan over the lanes with the chunk transfer P = M^per and its squares gives
// every chunk's start state, and the lane runs its blocks again from there,
// storing each block's start.  The serial depth is 2 per + 6 steps (a scan
// over groups of 64 blocks with a carry between them waits out a memory round
// trip per group: 14.4 us per pass at c4, 938 blocks per row).
constexpr int kPrefixWaves = 4;
constexpr int kPrefixHeld = 16;  // aggregates a lane keeps in registers

struct Mat2 {
    double a, b, c, d;  // row major
};

__device__ __forceinline__ Mat2 mat2_mul(const Mat2 &x, const Mat2 &y) {
    return {fma(x.a, y.a, x.b * y.c), fma(x.a, y.b, x.b * y.d), fma(x.c, y.a, x.d * y.c),
            fma(x.c, y.b, x.d * y.d)};
}

template <int NS>
__global__ void __launch_bounds__(kWave *kPrefixWaves)
    iir_prefix_kernel(const IirTable *__restrict__ table, double *__restrict__ aggr, int nblk,
                      int64_t nseq) {
    const IirTable &t = *table;
    const int64_t seq = int64_t(blockIdx.x) * kPrefixWaves +
                        __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x) / kWave);
    if (seq >= nseq) return;  // whole wavefronts only
    const int k = static_cast<int>(seq % NS);
    const int lane = threadIdx.x % kWave;
    double2 *agg = reinterpret_cast<double2 *>(aggr + seq * nblk * 2);
    const double *pm = t.pw[kLevelBlock][k];
    const Mat2 m{pm[0], pm[1], pm[2], pm[3]};
    const int per = (nblk + kWave - 1) / kWave;
    const int j0 = lane * per;
    const int j1 = j0 + per < nblk ? j0 + per : nblk;
    // the chunk's first kPrefixHeld aggregates stay in registers for both
    // runs (one memory round trip for chunks of up to kPrefixHeld blocks)
    double2 held[kPrefixHeld];
#pragma unroll
    for (int i = 0; i < kPrefixHeld; ++i) {
        const int j = j0 + i < j1 ? j0 + i : (j1 > 0 ? j1 - 1 : 0);
        held[i] = agg[j];
    }
    // the chunk's end state from a zero start
    double tu = 0.0, tv = 0.0;
#pragma unroll
    for (int i = 0; i < kPrefixHeld; ++i) {
        if (j0 + i < j1) {
            const double u = fma(m.a, tu, fma(m.b, tv, held[i].x));
            const double v = fma(m.c, tu, fma(m.d, tv, held[i].y));
            tu = u;
            tv = v;
        }
    }
#pragma unroll 4
    for (int j = j0 + kPrefixHeld; j < j1; ++j) {
        const double2 e = agg[j];
        const double u = fma(m.a, tu, fma(m.b, tv, e.x));
        const double v = fma(m.c, tu, fma(m.d, tv, e.y));
        tu = u;
        tv = v;
    }
    // P = M^per, square and multiply
    Mat2 q{1.0, 0.0, 0.0, 1.0}, sq = m;
    for (int e = per; e != 0; e >>= 1) {
        if (e & 1) q = mat2_mul(q, sq);
        sq = mat2_mul(sq, sq);
    }
    // inclusive scan of the chunk ends over the lanes, level j with P^(2^j)
#pragma unroll
    for (int j = 0; j < 6; ++j) {
        const int d = 1 << j;
        const double ou = shfl_up(tu, d), ov = shfl_up(tv, d);
        if (lane >= d) {
            tu = fma(q.a, ou, fma(q.b, ov, tu));
            tv = fma(q.c, ou, fma(q.d, ov, tv));
        }
        q = mat2_mul(q, q);
    }
    // the lane's start state is the end state of the chunks before it
    double su = shfl_up(tu, 1), sv = shfl_up(tv, 1);
    if (lane == 0) su = sv = 0.0;
#pragma unroll
    for (int i = 0; i < kPrefixHeld; ++i) {
        if (j0 + i < j1) {
            agg[j0 + i] = make_double2(su, sv);
            const double u = fma(m.a, su, fma(m.b, sv, held[i].x));
            const double v = fma(m.c, su, fma(m.d, sv, held[i].y));
            su = u;
            sv = v;
        }
    }
#pragma unroll 4
    for (int j = j0 + kPrefixHeld; j < j1; ++j) {
        const double2 e = agg[j];
        agg[j] = make_double2(su, sv);
        const double u = fma(m.a, su, fma(m.b, sv, e.x));
        const double v = fma(m.c, su, fma(m.d, sv, e.y));
        su = u;
        sv = v;
    }
}

template <int NA, int NB, class Mode, bool kLaneStates, int kPrefix, bool kWarmB = false>
__global__ void __launch_bounds__(kWave)
    iir_output_kernel(Mode m, const IirTable *__restrict__ table,
                      const double *__restrict__ aggr, const double *__restrict__ lanes,
                      int64_t len, int nblk) {
    constexpr int NS = NA + NB;
    static_assert(kLaneStates || kPrefix == kStoredStarts,
                  "grids that recompute the lane states take stored block starts");
    static_assert(!kWarmB || (kLaneStates && kPrefix != kStoredStarts && NB == 1),
                  "filter B warms up beside stored lane states of A and their block starts");
    const int row = blockIdx.x / nblk;
    const int blk = blockIdx.x - row * nblk;
    const int lane = threadIdx.x;
    const int64_t j0 = int64_t(blk) * kSpan + int64_t(lane) * kChunk;

    // everything this wavefront reads is requested up front: the block start
    // states, the lane start states, the row constants and the raw inputs
    const double *row_aggr = aggr + int64_t(row) * NS * nblk * 2;
    BankPair<NA, NB> p;
    Bank<NS> e0, e1;  // kFusedSums, kWindowStarts: the block aggregates this block starts from
    PairPowers<NS> pp;
    if constexpr (kPrefix == kFusedSums) {
        block_start_load<NS, kWarmB ? NA : NS>(row_aggr, nblk, blk, lane, e0, e1);
        pp.load(*table, lane);
    } else if constexpr (kPrefix == kWindowStarts) {
        block_window_load<NS, kWarmB ? NA : NS>(row_aggr, nblk, blk, e0, e1);
    } else {
#pragma unroll
        for (int k = 0; k < NS; ++k) {
            const double *src = row_aggr + (int64_t(k) * nblk + blk) * 2;
            p.u(k) = src[0];
            p.v(k) = src[1];
        }
    }
    BankPair<NA, NB> s;
    if constexpr (kLaneStates) {
        const double2 *src =
            reinterpret_cast<const double2 *>(lanes) + (int64_t(row) * nblk + blk) * NS * kWave;
#pragma unroll
        for (int k = 0; k < (kWarmB ? NA : NS); ++k) {
            const double2 w = src[k * kWave + lane];
            s.u(k) = w.x;
            s.v(k) = w.y;
        }
    }
    // kWarmB: filter B's inputs of this lane's chunks in the kWarmBlocks
    // blocks before this one (warm[w - 1] is block blk - w; before the row
    // start block 0 is read and not used), requested with the other loads
    typename Mode::In warm[kWarmB ? kWarmBlocks : 1][kChunk][Mode::kInputs];
    if constexpr (kWarmB) {
        // (B's filter input is the Mode's input 1 as it is: PipeBwdMode)
        static_assert(Mode::kInputs == 2, "filter B reads input 1");
        const typename Mode::In *b_src = m.src(row, 1);
#pragma unroll
        for (int w = 1; w <= kWarmBlocks; ++w) {
            const int64_t jw = blk - w >= 0 ? j0 - int64_t(w) * kSpan : int64_t(lane) * kChunk;
            const int64_t lo = chunk_lo<Mode::kReverse>(jw, len);  // full chunks
            typename Mode::In buf[kChunk];
#pragma unroll
            for (int r = 0; r < kChunk / 4; ++r) {
                __builtin_memcpy(buf + 4 * r, b_src + lo + 4 * r, 4 * sizeof(typename Mode::In));
            }
#pragma unroll
            for (int i = 0; i < kChunk; ++i) {
                warm[w - 1][i][0] = typename Mode::In(0);
                warm[w - 1][i][1] = buf[Mode::kReverse ? kChunk - 1 - i : i];
            }
        }
    }
    // the row constants' loads (Modes with Pre) go out before the raw
    // inputs', whose placement waits for every load issued before it: one
    // wait for all of them
    typename Mode::In in[kChunk][Mode::kInputs];
    double sh[4];
    if constexpr (HasPre<Mode>::value) {
        typename Mode::Pre pre;
        m.prefetch(row, lane, pre);
        load_chunk(m, row, j0, len, in);
        m.setup(row, sh, lane, pre);
    } else {
        load_chunk(m, row, j0, len, in);
        m.setup(row, sh, lane);
    }
    const IirTable &t2 = *table;
    if constexpr (kPrefix != kStoredStarts) {
        if constexpr (kPrefix == kFusedSums) {
            __shared__ double red[wave_sums_lds_doubles<2 * NS>()];
            block_start_reduce<NS>(t2, pp, e0, e1, red, lane);
        } else {
            block_window_start<NS>(t2, e0, e1);
        }
#pragma unroll
        for (int k = 0; k < NS; ++k) {
            p.u(k) = e0.u[k];
            p.v(k) = e0.v[k];
        }
    }
    if constexpr (kWarmB) {
        // filter B's block start state: its chunk end states from zero in
        // the previous blocks (weighted sums), v = sum_w M^(w - 1) e_(blk - w)
        // per lane (oldest block first), carried to the block end by
        // A^(kChunk (63 - lane)) and summed over the lanes in LDS
        Coeffs<NA, 0, Mode::kB2> none;
        Coeffs<NA, NB, Mode::kB2> wb;
        wb.load(t2, t2.c0b);
        const double *mk = t2.pw[kLevelBlock][NA];
        double vu = 0.0, vv = 0.0;
#pragma unroll
        for (int w = kWarmBlocks; w >= 1; --w) {
            if (blk - w < 0) continue;  // wave uniform
            const double u = vu, v = vv;
            vu = fma(mk[0], u, mk[1] * v);
            vv = fma(mk[2], u, mk[3] * v);
            BankPair<0, NB, NA> e;
            e.zero();
            zero_run<false, true>(m, t2, none, wb, warm[w - 1], j0 - int64_t(w) * kSpan, len, e);
            vu += e.b.u[0];
            vv += e.b.v[0];
        }
        __shared__ double red_b[wave_sums_lds_doubles<2>()];
        const double *lp = t2.lane_pw[NA][kWave - 1 - lane];
        const double wsum[2] = {fma(lp[0], vu, lp[1] * vv), fma(lp[2], vu, lp[3] * vv)};
        const double sum = wave_sums_lds(wsum, red_b, lane);  // component j in lane 4 j
        if (lane % 4 == 0 && lane / 4 < 2) red_b[lane / 4] = sum;
        wave_lds_fence();
        p.b.u[0] = red_b[0];
        p.b.v[0] = red_b[1];
        wave_lds_fence();
        // and its in-block lane start states, as the aggregate pass forms them
        BankPair<0, NB, NA> sb;
        sb.zero();
        if (general_chunk(j0, len)) {
            zero_run<true, false>(m, t2, none, wb, in, j0, len, sb);
        } else {
            zero_run<false, false>(m, t2, none, wb, in, j0, len, sb);
        }
        sb.scan_chunks(t2, lane);
        s.b.u[0] = dpp_move<0x138, 0xF>(sb.b.u[0]);  // wave_shr:1 (lane 0 reads 0)
        s.b.v[0] = dpp_move<0x138, 0xF>(sb.b.v[0]);
    }
    if constexpr (!kLaneStates) {
        // the in-block start states again: zero state run, scan, shift by a lane
        Coeffs<0, NA, Mode::kB2> za;
        Coeffs<NA, NB, Mode::kB2> zb;
        za.load(t2, t2.c0a);
        zb.load(t2, t2.c0b);
        s.zero();
        if (general_chunk(j0, len)) {
            zero_run<true, true>(m, t2, za, zb, in, j0, len, s);
        } else {
            zero_run<false, true>(m, t2, za, zb, in, j0, len, s);
        }
        s.scan_chunks(t2, lane);
#pragma unroll
        for (int k = 0; k < NS; ++k) {
            s.u(k) = dpp_move<0x138, 0xF>(s.u(k));
            s.v(k) = dpp_move<0x138, 0xF>(s.v(k));
        }
    }

    // lane start state = (start state given a zero block start) + A^(kChunk lane) p
#pragma unroll
    for (int k = 0; k < NS; ++k) {
        const double *lp = t2.lane_pw[k][lane];
        const double pu = p.u(k), pv = p.v(k);
        s.u(k) = fma(lp[0], pu, fma(lp[1], pv, s.u(k)));
        s.v(k) = fma(lp[2], pu, fma(lp[3], pv, s.v(k)));
    }

    // run from the true start state
    Coeffs<0, NA, Mode::kB2> ca;
    Coeffs<NA, NB, Mode::kB2> cb;
    ca.load(t2, t2.c0a);
    cb.load(t2, t2.c0b);
    typename Mode::Out out[Mode::kOutputs][kChunk];
    double acc = 0.0;
    if (general_chunk(j0, len)) {
        output_run<true>(m, ca, cb, in, j0, len, sh, s, out, acc);
    } else {
        output_run<false>(m, ca, cb, in, j0, len, sh, s, out, acc);
    }
#pragma unroll
    for (int q = 0; q < Mode::kOutputs; ++q) {
        typename Mode::Out *dst = m.dst(row, q);
        if (dst != nullptr) store_chunk(dst, out[q], Mode::kReverse, j0, len);
    }

    if constexpr (Mode::kAccumulates) {
        acc = wave_sum(acc);
        if (lane == 0) m.finish(row, blk, acc);
    }
}

// ---------------------------------------------------------------------------
// The output pass of lane-state grids with windowed block starts by
// kOutputWaves wavefronts per block, each on its own sections (as the split
// aggregate pass).  Filter A's sections are shared out in order over the
// first OutputSplit::kAWaves wavefronts; the last wavefront also runs filter
// B (with kWarmB, whose warm-up is the longest chain, it runs filter B alone)
// and forms the Mode's outputs.  A's output c0 x + y_0 + ... + y_(NA-1) is
// summed in section order as Coeffs::step sums it: the first wavefront's
// running sums go through LDS to the next, which adds its sections' outputs,
// and so on to the last, so the outputs are bitwise those of the one-wavefront
// pass (iir_output_kernel).  The pipeline launches it for the backward's
// output pass with filter B's warm-up (kWarmB, two wavefronts: the level
// alignment filter on one, the pre-emphasis filter's warm-up, lane scan and
// recursion on the other, where one wavefront ran both in turn); the forward's
// output pass split over two or three wavefronts was no faster in the step.
// ---------------------------------------------------------------------------
template <int NA, int NB, bool kWarmB>
struct OutputSplit {
    static constexpr int kAWaves = kWarmB ? kOutputWaves - 1 : kOutputWaves;
    static constexpr int kPer = (NA + kAWaves - 1) / kAWaves;
    // filter A's sections of wavefront w: [lo(w), hi(w))
    static constexpr int lo(int w) { return w * kPer < NA ? w * kPer : NA; }
    static constexpr int hi(int w) { return w == kOutputWaves - 1 ? NA : lo(w + 1); }
    // every A wavefront has a section
    static constexpr bool kValid = kAWaves >= 1 && (kAWaves - 1) * kPer < NA;
};

// The recursion of one wavefront's sections over its lane's chunk: with
// kFirst the running sums c0 x + y_lo + ... (yrun), else each A section's
// output (ya[k]); with B sections B's output (yb, Coeffs::step).
template <bool kGeneral, bool kFirst, int A0, int NAW, int NBW, class Mode>
__device__ __forceinline__ void split_run(const Mode &m, const Coeffs<A0, NAW, Mode::kB2> &ca,
                                          const Coeffs<A0 + NAW, NBW, Mode::kB2> &cb,
                                          const typename Mode::In (&in)[kChunk][Mode::kInputs],
                                          int64_t j0, int64_t len, BankPair<NAW, NBW, A0> &s,
                                          double (&yrun)[kChunk],
                                          double (&ya)[NAW > 0 ? NAW : 1][kChunk],
                                          double (&yb)[kChunk]) {
#pragma unroll
    for (int i = 0; i < kChunk; ++i) {
        double w, xa, xb;
        element_inputs<kGeneral>(m, in[i], j0 + i, len, w, xa, xb);
        if constexpr (kFirst) {
            yrun[i] = ca.step(s.a, xa);
        } else if constexpr (NAW > 0) {
            double y[NAW];
            ca.step_parts(s.a, xa, y);
#pragma unroll
            for (int k = 0; k < NAW; ++k) ya[k][i] = y[k];
        }
        if constexpr (NBW > 0) yb[i] = cb.step(s.b, xb);
    }
}

// the Mode's outputs of the lane's chunk from A's and B's outputs (the last
// wavefront), as output_run forms them
template <bool kGeneral, class Mode>
__device__ __forceinline__ void split_finish(const Mode &m,
                                             const typename Mode::In (&in)[kChunk][Mode::kInputs],
                                             int64_t j0, int64_t len, const double *sh,
                                             const double (&ya)[kChunk], const double (&yb)[kChunk],
                                             typename Mode::Out (&out)[Mode::kOutputs][kChunk],
                                             double &acc) {
#pragma unroll
    for (int i = 0; i < kChunk; ++i) {
        const int64_t j = j0 + i;
        double w, xa, xb;
        element_inputs<kGeneral>(m, in[i], j, len, w, xa, xb);
        typename Mode::Out o[Mode::kOutputs];
        const double before = acc;
        m.compute(w, ya[i], yb[i], acc, sh, o);
        if constexpr (kGeneral) {
            if (j >= len) acc = before;  // past the end of the row
        }
#pragma unroll
        for (int q = 0; q < Mode::kOutputs; ++q) {
            out[q][i] = (!kGeneral || j < len) ? o[q] : typename Mode::Out(0);
        }
    }
}

template <int NA, int NB, class Mode, bool kWarmB, int W>
__device__ __forceinline__ void output_split_wave(const Mode &m, const IirTable &t,
                                                  const double *aggr, const double *lanes,
                                                  int64_t len, int nblk, int row, int blk,
                                                  int lane, int w, double *run) {
    if (w != W) {
        if constexpr (W + 1 < kOutputWaves) {
            output_split_wave<NA, NB, Mode, kWarmB, W + 1>(m, t, aggr, lanes, len, nblk, row,
                                                            blk, lane, w, run);
        }
        return;
    }
    using Plan = OutputSplit<NA, NB, kWarmB>;
    static_assert(Plan::kValid, "every A wavefront has a section");
    constexpr int NS = NA + NB;
    constexpr bool kLast = W == kOutputWaves - 1;
    constexpr int A0 = Plan::lo(W);
    constexpr int NAW = Plan::hi(W) - A0;  // filter A's sections here
    constexpr int NBW = kLast ? NB : 0;    // filter B's sections here
    constexpr int N = NAW + NBW;           // sections A0 .. A0 + N - 1
    constexpr int NL = kWarmB && kLast ? NAW : N;  // of them with aggregates and lane states
    static_assert(!kWarmB || (NB == 1 && Mode::kInputs == 2), "filter B warms up on input 1");
    static_assert(!kWarmB || !kLast || NAW == 0, "with kWarmB filter B has a wavefront alone");
    const int64_t j0 = int64_t(blk) * kSpan + int64_t(lane) * kChunk;

    // this wavefront's loads, all requested before the first wait: the
    // aggregates of the two blocks before this one, the lane states, filter
    // B's warm-up inputs, the row constants and the raw inputs
    Bank<N> e0, e1;
    block_window_load<N, NL>(aggr + (int64_t(row) * NS + A0) * nblk * 2, nblk, blk, e0, e1);
    BankPair<NAW, NBW, A0> s;
    {
        const double2 *src = reinterpret_cast<const double2 *>(lanes) +
                             ((int64_t(row) * nblk + blk) * NS + A0) * kWave;
#pragma unroll
        for (int k = 0; k < NL; ++k) {
            const double2 v = src[k * kWave + lane];
            s.u(k) = v.x;
            s.v(k) = v.y;
        }
    }
    typename Mode::In warm[kWarmB && kLast ? kWarmBlocks : 1][kChunk][Mode::kInputs];
    if constexpr (kWarmB && kLast) {
        const typename Mode::In *b_src = m.src(row, 1);
#pragma unroll
        for (int q = 1; q <= kWarmBlocks; ++q) {
            const int64_t jw = blk - q >= 0 ? j0 - int64_t(q) * kSpan : int64_t(lane) * kChunk;
            const int64_t lo = chunk_lo<Mode::kReverse>(jw, len);  // full chunks
            typename Mode::In buf[kChunk];
#pragma unroll
            for (int r = 0; r < kChunk / 4; ++r) {
                __builtin_memcpy(buf + 4 * r, b_src + lo + 4 * r, 4 * sizeof(typename Mode::In));
            }
#pragma unroll
            for (int i = 0; i < kChunk; ++i) {
                warm[q - 1][i][0] = typename Mode::In(0);
                warm[q - 1][i][1] = buf[Mode::kReverse ? kChunk - 1 - i : i];
            }
        }
    }
    typename Mode::In in[kChunk][Mode::kInputs];
    double sh[4];
    if constexpr (kLast && HasPre<Mode>::value) {
        typename Mode::Pre pre;
        m.prefetch(row, lane, pre);
        load_chunk(m, row, j0, len, in);
        m.setup(row, sh, lane, pre);
    } else {
        load_chunk(m, row, j0, len, in);
        if constexpr (kLast) m.setup(row, sh, lane);
    }

    // block start states (windowed), filter B's by warm-up
    BankPair<NAW, NBW, A0> p;
    block_window_start<N, A0>(t, e0, e1);
#pragma unroll
    for (int k = 0; k < N; ++k) {
        p.u(k) = e0.u[k];
        p.v(k) = e0.v[k];
    }
    if constexpr (kWarmB && kLast) {
        // as iir_output_kernel: filter B's chunk end states from zero in the
        // previous blocks, carried to this block's start and summed in LDS,
        // then its in-block lane start states by the aggregate pass's steps
        Coeffs<A0, 0, Mode::kB2> none;
        Coeffs<A0, NBW, Mode::kB2> wb;
        wb.load(t, t.c0b);
        const double *mk = t.pw[kLevelBlock][NA];
        double vu = 0.0, vv = 0.0;
#pragma unroll
        for (int q = kWarmBlocks; q >= 1; --q) {
            if (blk - q < 0) continue;  // wave uniform
            const double u = vu, v = vv;
            vu = fma(mk[0], u, mk[1] * v);
            vv = fma(mk[2], u, mk[3] * v);
            BankPair<0, NBW, A0> e;
            e.zero();
            zero_run<false, true>(m, t, none, wb, warm[q - 1], j0 - int64_t(q) * kSpan, len, e);
            vu += e.b.u[0];
            vv += e.b.v[0];
        }
        __shared__ double red_b[wave_sums_lds_doubles<2>()];
        const double *lp = t.lane_pw[NA][kWave - 1 - lane];
        const double wsum[2] = {fma(lp[0], vu, lp[1] * vv), fma(lp[2], vu, lp[3] * vv)};
        const double sum = wave_sums_lds(wsum, red_b, lane);  // component j in lane 4 j
        if (lane % 4 == 0 && lane / 4 < 2) red_b[lane / 4] = sum;
        wave_lds_fence();
        p.b.u[0] = red_b[0];
        p.b.v[0] = red_b[1];
        wave_lds_fence();
        BankPair<0, NBW, A0> sb;
        sb.zero();
        if (general_chunk(j0, len)) {
            zero_run<true, false>(m, t, none, wb, in, j0, len, sb);
        } else {
            zero_run<false, false>(m, t, none, wb, in, j0, len, sb);
        }
        sb.scan_chunks(t, lane);
        s.b.u[0] = dpp_move<0x138, 0xF>(sb.b.u[0]);  // wave_shr:1 (lane 0 reads 0)
        s.b.v[0] = dpp_move<0x138, 0xF>(sb.b.v[0]);
    }
    // lane start state = (start state given a zero block start) + A^(kChunk lane) p
#pragma unroll
    for (int k = 0; k < N; ++k) {
        const double *lp = t.lane_pw[A0 + k][lane];
        const double pu = p.u(k), pv = p.v(k);
        s.u(k) = fma(lp[0], pu, fma(lp[1], pv, s.u(k)));
        s.v(k) = fma(lp[2], pu, fma(lp[3], pv, s.v(k)));
    }

    // the recursion over this wavefront's sections
    Coeffs<A0, NAW, Mode::kB2> ca;
    Coeffs<A0 + NAW, NBW, Mode::kB2> cb;
    ca.load(t, W == 0 ? t.c0a : 0.0);
    if constexpr (NBW > 0) cb.load(t, t.c0b);
    double yrun[kChunk], ya[NAW > 0 ? NAW : 1][kChunk], yb[kChunk];
    if (general_chunk(j0, len)) {
        split_run<true, W == 0>(m, ca, cb, in, j0, len, s, yrun, ya, yb);
    } else {
        split_run<false, W == 0>(m, ca, cb, in, j0, len, s, yrun, ya, yb);
    }

    // A's running sums from wavefront to wavefront (run is [kChunk][kWave]).
    // The barriers sit in wavefront specific code, but the branch to it is
    // uniform per wavefront and every wavefront passes all kOutputWaves - 1
    // of them, in the same order, outside any lane divergent branch, so each
    // s_barrier is met by the whole workgroup.
#pragma unroll
    for (int b = 1; b < kOutputWaves; ++b) {
        if (W == b - 1) {
#pragma unroll
            for (int i = 0; i < kChunk; ++i) run[i * kWave + lane] = yrun[i];
        }
        __syncthreads();
        if (W == b) {
#pragma unroll
            for (int i = 0; i < kChunk; ++i) {
                double y = run[i * kWave + lane];
#pragma unroll
                for (int k = 0; k < NAW; ++k) y += ya[k][i];
                yrun[i] = y;
            }
        }
    }

    if constexpr (kLast) {
        typename Mode::Out out[Mode::kOutputs][kChunk];
        double acc = 0.0;
        if (general_chunk(j0, len)) {
            split_finish<true>(m, in, j0, len, sh, yrun, yb, out, acc);
        } else {
            split_finish<false>(m, in, j0, len, sh, yrun, yb, out, acc);
        }
#pragma unroll
        for (int q = 0; q < Mode::kOutputs; ++q) {
            typename Mode::Out *dst = m.dst(row, q);
            if (dst != nullptr) store_chunk(dst, out[q], Mode::kReverse, j0, len);
        }
        if constexpr (Mode::kAccumulates) {
            acc = wave_sum(acc);
            if (lane == 0) m.finish(row, blk, acc);
        }
    }
}

template <int NA, int NB, class Mode, bool kWarmB>
__global__ void __launch_bounds__(kOutputWaves * kWave)
    iir_output_split_kernel(Mode m, const IirTable *__restrict__ table,
                            const double *__restrict__ aggr, const double *__restrict__ lanes,
                            int64_t len, int nblk) {
    __shared__ double run[kChunk * kWave];
    const int row = blockIdx.x / nblk;
    const int blk = blockIdx.x - row * nblk;
    output_split_wave<NA, NB, Mode, kWarmB, 0>(m, *table, aggr, lanes, len, nblk, row, blk,
                                               static_cast<int>(threadIdx.x) % kWave,
                                               wave_index(), run);
}

// Host side: aggregate, prefix and output launches of one scan pass over
// `rows` rows; `ws` holds scan_workspace_doubles(rows, nblk, NA + NB).
// split: the aggregate pass of lane-state grids by kSplitWaves wavefronts per
// block (iir_aggregate_split_kernel).  window: the table's sections decay
// below kWindowDecay over kWarmBlocks blocks (the caller has checked it), so
// the output pass of lane-state grids takes windowed block starts (no prefix
// pass).  warm_b (lane-state grids with windowed or fused block starts): the
// output pass warms filter B up itself, the aggregate pass need not have run
// it.
template <int NA, int NB, class Mode>
int launch_scan(const Mode &m, const IirTable *table, double *ws, int64_t rows, int64_t len,
                bool aggregate, bool output, hipStream_t stream, bool split = false,
                bool warm_b = false, bool window = false) {
    constexpr int NS = NA + NB;
    static_assert(NS <= kMaxSections, "too many sections");
    const int64_t nblk = cdiv(len, kBlockSpan);
    double *aggr = ws;
    double *lanes = ws + scan_aggr_doubles(rows, nblk, NS);
    const unsigned grid = static_cast<unsigned>(rows * nblk);
    if (grid == 0) return PESQ_OK;
    const ScanPlan plan = scan_plan(rows, nblk);
    const bool lane_states = plan.lane_states;
    const bool windowed = window && lane_states;
    const bool fused = !windowed && plan.fused_prefix;
    PESQ_CHECK_ARG(!warm_b || (NB == 1 && Mode::kInputs == 2 && (windowed || fused)),
                   "filter B warms up only beside windowed or fused block starts");
    if (aggregate) {
        bool launched = false;
        if constexpr (NA + NB >= kSplitWaves) {
            if (lane_states && split) {
                hipLaunchKernelGGL((iir_aggregate_split_kernel<NA, NB, kSplitWaves, Mode>),
                                   dim3(grid), dim3(kSplitWaves * kWave), 0, stream, m, table,
                                   aggr, lanes, len, static_cast<int>(nblk));
                launched = true;
            }
        }
        if (launched) {
        } else if (lane_states) {
            hipLaunchKernelGGL((iir_aggregate_kernel<NA, NB, Mode, true>), dim3(grid), dim3(kWave),
                               0, stream, m, table, aggr, lanes, len, static_cast<int>(nblk));
        } else {
            hipLaunchKernelGGL((iir_aggregate_kernel<NA, NB, Mode, false>), dim3(grid),
                               dim3(kWave), 0, stream, m, table, aggr, lanes, len,
                               static_cast<int>(nblk));
        }
        PESQ_CHECK_LAUNCH("iir aggregate");
        if (!fused && !windowed) {
            const int64_t nseq = rows * NS;
            hipLaunchKernelGGL(iir_prefix_kernel<NS>,
                               dim3(static_cast<unsigned>(cdiv(nseq, kPrefixWaves))),
                               dim3(kWave * kPrefixWaves), 0, stream, table, aggr,
                               static_cast<int>(nblk), nseq);
            PESQ_CHECK_LAUNCH("iir prefix");
        }
    }
    if (output) {
        const double *ca = aggr;
        const double *cl = lanes;
        const int nb = static_cast<int>(nblk);
        bool launched = false;
        if constexpr (kSplitOutput && NB == 1 && Mode::kInputs == 2 &&
                      OutputSplit<NA, NB, true>::kValid) {
            if (windowed && warm_b) {
                hipLaunchKernelGGL((iir_output_split_kernel<NA, NB, Mode, true>), dim3(grid),
                                   dim3(kOutputWaves * kWave), 0, stream, m, table, ca, cl, len,
                                   nb);
                launched = true;
            }
        }
        if constexpr (NB == 1 && Mode::kInputs == 2) {
            // filter B's block starts from its own warm-up (no aggregates of B)
            if (launched) {
            } else if (windowed && warm_b) {
                hipLaunchKernelGGL((iir_output_kernel<NA, NB, Mode, true, kWindowStarts, true>),
                                   dim3(grid), dim3(kWave), 0, stream, m, table, ca, cl, len, nb);
                launched = true;
            } else if (fused && warm_b) {
                hipLaunchKernelGGL((iir_output_kernel<NA, NB, Mode, true, kFusedSums, true>),
                                   dim3(grid), dim3(kWave), 0, stream, m, table, ca, cl, len, nb);
                launched = true;
            }
        }
        if (launched) {
        } else if (windowed) {
            hipLaunchKernelGGL((iir_output_kernel<NA, NB, Mode, true, kWindowStarts>),
                               dim3(grid), dim3(kWave), 0, stream, m, table, ca, cl, len, nb);
        } else if (fused) {
            hipLaunchKernelGGL((iir_output_kernel<NA, NB, Mode, true, kFusedSums>), dim3(grid),
                               dim3(kWave), 0, stream, m, table, ca, cl, len, nb);
        } else if (lane_states) {
            hipLaunchKernelGGL((iir_output_kernel<NA, NB, Mode, true, kStoredStarts>),
                               dim3(grid), dim3(kWave), 0, stream, m, table, ca, cl, len, nb);
        } else {
            hipLaunchKernelGGL((iir_output_kernel<NA, NB, Mode, false, kStoredStarts>),
                               dim3(grid), dim3(kWave), 0, stream, m, table, ca, cl, len, nb);
        }
        PESQ_CHECK_LAUNCH("iir output");
    }
    return PESQ_OK;
}

}  // namespace pesq
