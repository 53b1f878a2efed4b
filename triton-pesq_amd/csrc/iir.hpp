// Chunked parallel scan of a bank of parallel second order sections, fp64 state.
//
// A filter is realised in parallel form, y = c0 x + sum_k y_k, where section k
// is a direct form II transposed biquad
//     y_k  = b0 x + z1
//     z1'  = b1 x - a1 y_k + z2
//     z2'  = b2 x - a2 y_k
// i.e. the state z = (z1, z2) evolves as z' = A_k z + beta_k x with
// A_k = [[-a1, 1], [-a2, 0]].  Because every A_k is 2x2 and the sections are
// independent, the chunk transfer matrices are block diagonal (4 numbers per
// section) and the scan combine costs 4 FMAs per section.
//
// Geometry: one lane runs the recursion over a chunk of kChunk samples; a
// wavefront covers 64 consecutive chunks, a workgroup kWaves wavefronts (one
// "block" of kBlockSpan samples).  Two kernels per pass:
//   aggregate: zero state run per chunk, in-wave Kogge-Stone scan, block end
//              state written to `aggr` (the block's contribution to the state
//              after it, given a zero state before it);
//   output:    zero state run, in-wave scan, block start state from a scan of
//              the preceding blocks' aggregates, lane start state, re-run of
//              the recursion from it, outputs.
// The time axis can be reversed (adjoint filter) by the Mode policy.
//
// Two filters (A and B) can be scanned in the same pass on different inputs;
// the pipeline uses this to run the level-alignment band pass and the
// pre-emphasis filter together.
#pragma once

#include "common.hpp"

namespace pesq {

constexpr int kChunk = 16;                      // samples per lane
constexpr int kWaves = 4;                       // wavefronts per workgroup
constexpr int kBlockChunks = kWave * kWaves;    // chunks per workgroup
constexpr int64_t kBlockSpan = int64_t(kBlockChunks) * kChunk;  // samples per workgroup
constexpr int kMaxSections = PESQ_IIR_MAX_SECTIONS;
// power levels: A^(kChunk * 2^j); j = 0..5 in-wave, 6 = one wave, 8 = one
// block (kBlockChunks = 2^8 chunks), 8..13 = the block level scan
constexpr int kLevelWave = 6;
constexpr int kLevelBlock = 8;
constexpr int kLevels = 14;
static_assert(kBlockChunks == (1 << kLevelBlock), "block must be 2^8 chunks");

struct IirTable {
    int32_t na, nb;      // sections of filter A, then of filter B
    double c0a, c0b;     // direct feed through of A and B
    double b0[kMaxSections], b1[kMaxSections], b2[kMaxSections];
    double a1[kMaxSections], a2[kMaxSections];
    double pw[kLevels][kMaxSections][4];  // A_k^(kChunk 2^j), row major 2x2
};

// --------------------------------------------------------------------------
// per lane state of a bank of NS sections starting at section S0
// --------------------------------------------------------------------------

template <int NS>
struct Bank {
    double z[NS > 0 ? NS : 1][2];

    __device__ __forceinline__ void zero() {
#pragma unroll
        for (int k = 0; k < NS; ++k) z[k][0] = z[k][1] = 0.0;
    }
};

template <int S0, int NS>
struct Coeffs {
    double b0[NS > 0 ? NS : 1], b1[NS > 0 ? NS : 1], b2[NS > 0 ? NS : 1];
    double a1[NS > 0 ? NS : 1], a2[NS > 0 ? NS : 1];
    double c0;

    __device__ __forceinline__ void load(const IirTable &t, double direct) {
#pragma unroll
        for (int k = 0; k < NS; ++k) {
            b0[k] = t.b0[S0 + k];
            b1[k] = t.b1[S0 + k];
            b2[k] = t.b2[S0 + k];
            a1[k] = t.a1[S0 + k];
            a2[k] = t.a2[S0 + k];
        }
        c0 = direct;
    }

    // one time step: consumes x, advances the state, returns the output
    __device__ __forceinline__ double step(Bank<NS> &s, double x) const {
        double y = c0 * x;
#pragma unroll
        for (int k = 0; k < NS; ++k) {
            const double yk = fma(b0[k], x, s.z[k][0]);
            s.z[k][0] = fma(-a1[k], yk, fma(b1[k], x, s.z[k][1]));
            s.z[k][1] = fma(-a2[k], yk, b2[k] * x);
            y += yk;
        }
        return y;
    }
};

// z <- P z + add, P = A^(kChunk 2^level) per section
template <int S0, int NS>
__device__ __forceinline__ void apply_power(const IirTable &t, int level, Bank<NS> &z,
                                            const Bank<NS> &add) {
#pragma unroll
    for (int k = 0; k < NS; ++k) {
        const double *p = t.pw[level][S0 + k];
        const double u = z.z[k][0], v = z.z[k][1];
        z.z[k][0] = fma(p[0], u, fma(p[1], v, add.z[k][0]));
        z.z[k][1] = fma(p[2], u, fma(p[3], v, add.z[k][1]));
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
            o.z[k][0] = shfl_up(z.z[k][0], d);
            o.z[k][1] = shfl_up(z.z[k][1], d);
        }
        if (lane >= d) {
            // z <- z + P o, written as o <- P o + z then copy
            apply_power<S0, NS>(t, level0 + j, o, z);
#pragma unroll
            for (int k = 0; k < NS; ++k) {
                z.z[k][0] = o.z[k][0];
                z.z[k][1] = o.z[k][1];
            }
        }
    }
}

template <int NS>
__device__ __forceinline__ void shift_up_one(Bank<NS> &z, int lane) {
#pragma unroll
    for (int k = 0; k < NS; ++k) {
        const double u = shfl_up(z.z[k][0], 1), v = shfl_up(z.z[k][1], 1);
        z.z[k][0] = lane == 0 ? 0.0 : u;
        z.z[k][1] = lane == 0 ? 0.0 : v;
    }
}

// --------------------------------------------------------------------------
// the two kernels, parametrised by a Mode policy:
//   Mode::kInputs                 number of float inputs per sample (1 or 2)
//   Mode::kReverse                process the time axis back to front
//   Mode::kAccumulates            the output pass reduces a per block sum
//   m.load(row, n, in[])          raw inputs at physical sample n
//   m.inputs(n, in[], xa, xb)     filter inputs from the raw ones
//   m.observe(o, in[]) / reduce_observed / combine_observed / observed(row, blk, o)
//                                 aggregate-pass reduction over the raw inputs
//   m.setup(row, blk, sh, lane)   output pass, wavefront 0 before the block
//                                 barrier: per row constants into sh[0..3]
//   m.emit(row, n, ya, yb, acc, sh) consume the outputs of sample n
//   m.finish(row, blk, total)     block total of the accumulator
// The scan itself is linear, so it runs in the units of the raw inputs and a
// per row normalisation is applied by emit.
// --------------------------------------------------------------------------

template <int NA, int NB>
struct BankPair {
    Bank<NA> a;
    Bank<NB> b;
};

template <int NA, int NB>
__device__ __forceinline__ void store_state(double *dst, const BankPair<NA, NB> &s) {
#pragma unroll
    for (int k = 0; k < NA; ++k) {
        dst[2 * k] = s.a.z[k][0];
        dst[2 * k + 1] = s.a.z[k][1];
    }
#pragma unroll
    for (int k = 0; k < NB; ++k) {
        dst[2 * (NA + k)] = s.b.z[k][0];
        dst[2 * (NA + k) + 1] = s.b.z[k][1];
    }
}

template <int NA, int NB>
__device__ __forceinline__ void load_state(BankPair<NA, NB> &s, const double *src, double scale) {
#pragma unroll
    for (int k = 0; k < NA; ++k) {
        s.a.z[k][0] = src[2 * k] * scale;
        s.a.z[k][1] = src[2 * k + 1] * scale;
    }
#pragma unroll
    for (int k = 0; k < NB; ++k) {
        s.b.z[k][0] = src[2 * (NA + k)] * scale;
        s.b.z[k][1] = src[2 * (NA + k) + 1] * scale;
    }
}

template <int NA, int NB>
__device__ __forceinline__ void scan_pair(const IirTable &t, int level0, BankPair<NA, NB> &s,
                                          int lane) {
    if constexpr (NA > 0) scan_wave<0, NA>(t, level0, s.a, lane);
    if constexpr (NB > 0) scan_wave<NA, NB>(t, level0, s.b, lane);
}

template <int NA, int NB>
__device__ __forceinline__ void power_pair(const IirTable &t, int level, BankPair<NA, NB> &s,
                                           const BankPair<NA, NB> &add) {
    if constexpr (NA > 0) apply_power<0, NA>(t, level, s.a, add.a);
    if constexpr (NB > 0) apply_power<NA, NB>(t, level, s.b, add.b);
}

template <int NA, int NB>
__device__ __forceinline__ void zero_pair(BankPair<NA, NB> &s) {
    s.a.zero();
    s.b.zero();
}

template <int NA, int NB, class Mode>
__global__ void __launch_bounds__(kWave *kWaves)
    iir_aggregate_kernel(Mode m, const IirTable *__restrict__ table, double *__restrict__ aggr,
                         int64_t len, int nblk) {
    constexpr int NSTATE = 2 * (NA + NB);
    __shared__ double totals[kWaves][NSTATE];
    __shared__ float observed[kWaves];

    const IirTable &t = *table;
    const int row = blockIdx.x / nblk;
    const int blk = blockIdx.x - row * nblk;
    const int wave = threadIdx.x / kWave;
    const int lane = threadIdx.x % kWave;
    const int64_t j0 = (int64_t(blk) * kBlockChunks + wave * kWave + lane) * kChunk;

    Coeffs<0, NA> ca;
    Coeffs<NA, NB> cb;
    ca.load(t, t.c0a);
    cb.load(t, t.c0b);

    BankPair<NA, NB> s;
    zero_pair(s);
    float obs = 0.0f;

#pragma unroll
    for (int i = 0; i < kChunk; ++i) {
        const int64_t j = j0 + i;
        float in[Mode::kInputs];
        double xa = 0.0, xb = 0.0;
        if (j < len) {
            const int64_t n = Mode::kReverse ? len - 1 - j : j;
            m.load(row, n, in);
            m.inputs(n, in, xa, xb);
            obs = m.observe(obs, in);
        }
        if constexpr (NA > 0) ca.step(s.a, xa);
        if constexpr (NB > 0) cb.step(s.b, xb);
    }

    scan_pair(t, 0, s, lane);
    if (lane == kWave - 1) store_state(totals[wave], s);
    obs = m.reduce_observed(obs);
    if (lane == 0) observed[wave] = obs;
    __syncthreads();

    if (threadIdx.x == 0) {
        BankPair<NA, NB> acc, w;
        load_state(acc, totals[0], 1.0);
        for (int i = 1; i < kWaves; ++i) {
            load_state(w, totals[i], 1.0);
            power_pair(t, kLevelWave, acc, w);
        }
        store_state(aggr + (int64_t(row) * nblk + blk) * NSTATE, acc);
        float o = observed[0];
        for (int i = 1; i < kWaves; ++i) o = m.combine_observed(o, observed[i]);
        m.observed(row, blk, o);
    }
}

template <int NA, int NB, class Mode>
__global__ void __launch_bounds__(kWave *kWaves)
    iir_output_kernel(Mode m, const IirTable *__restrict__ table,
                      const double *__restrict__ aggr, int64_t len, int nblk) {
    constexpr int NSTATE = 2 * (NA + NB);
    __shared__ double totals[kWaves][NSTATE];
    __shared__ double prefix[NSTATE];
    __shared__ double accum[kWaves];
    __shared__ double consts[4];

    const IirTable &t = *table;
    const int row = blockIdx.x / nblk;
    const int blk = blockIdx.x - row * nblk;
    const int wave = threadIdx.x / kWave;
    const int lane = threadIdx.x % kWave;
    const int64_t j0 = (int64_t(blk) * kBlockChunks + wave * kWave + lane) * kChunk;

    Coeffs<0, NA> ca;
    Coeffs<NA, NB> cb;
    ca.load(t, t.c0a);
    cb.load(t, t.c0b);

    // raw inputs of the chunk stay in registers for the second run
    float in[kChunk][Mode::kInputs];
#pragma unroll
    for (int i = 0; i < kChunk; ++i) {
        const int64_t j = j0 + i;
        if (j < len) {
            m.load(row, Mode::kReverse ? len - 1 - j : j, in[i]);
        } else {
#pragma unroll
            for (int q = 0; q < Mode::kInputs; ++q) in[i][q] = 0.0f;
        }
    }

    // zero state run -> chunk end state
    BankPair<NA, NB> s;
    zero_pair(s);
#pragma unroll
    for (int i = 0; i < kChunk; ++i) {
        const int64_t j = j0 + i;
        double xa = 0.0, xb = 0.0;
        if (j < len) m.inputs(Mode::kReverse ? len - 1 - j : j, in[i], xa, xb);
        if constexpr (NA > 0) ca.step(s.a, xa);
        if constexpr (NB > 0) cb.step(s.b, xb);
    }

    scan_pair(t, 0, s, lane);  // s = inclusive end state of the wave's chunks
    if (lane == kWave - 1) store_state(totals[wave], s);

    // state at the start of this block: scan of the preceding blocks' aggregates
    if (wave == 0) {
        BankPair<NA, NB> carry;
        zero_pair(carry);
        for (int base = 0; base < blk; base += kWave) {
            BankPair<NA, NB> v, zero;
            zero_pair(zero);
            const int jb = base + lane;
            if (jb < blk) {
                load_state(v, aggr + (int64_t(row) * nblk + jb) * NSTATE, 1.0);
            } else {
                zero_pair(v);
            }
            // element 0 also carries the state entering the tile
            BankPair<NA, NB> injected = carry;
            power_pair(t, kLevelBlock, injected, zero);
            if (lane == 0) {
                if constexpr (NA > 0) {
#pragma unroll
                    for (int k = 0; k < NA; ++k) {
                        v.a.z[k][0] += injected.a.z[k][0];
                        v.a.z[k][1] += injected.a.z[k][1];
                    }
                }
                if constexpr (NB > 0) {
#pragma unroll
                    for (int k = 0; k < NB; ++k) {
                        v.b.z[k][0] += injected.b.z[k][0];
                        v.b.z[k][1] += injected.b.z[k][1];
                    }
                }
            }
            scan_pair(t, kLevelBlock, v, lane);
            // state at the end of block min(blk, base + 64) - 1
            const int src = (blk - base < kWave ? blk - base : kWave) - 1;
            double flat[NSTATE];
            store_state(flat, v);
#pragma unroll
            for (int q = 0; q < NSTATE; ++q) flat[q] = shfl(flat[q], src);
            load_state(carry, flat, 1.0);
        }
        if (lane == 0) store_state(prefix, carry);
        m.setup(row, blk, consts, lane);
    }
    __syncthreads();

    // state entering this wave: the block prefix advanced over earlier waves
    BankPair<NA, NB> p;
    load_state(p, prefix, 1.0);
    for (int i = 0; i < wave; ++i) {
        BankPair<NA, NB> tot;
        load_state(tot, totals[i], 1.0);
        power_pair(t, kLevelWave, p, tot);
    }

    // lane start state = A^(lane L) p + (inclusive end state of lane - 1)
    BankPair<NA, NB> e;
    if (lane == 0) {
        e = p;
    } else {
        zero_pair(e);
    }
    scan_pair(t, 0, e, lane);
    if constexpr (NA > 0) shift_up_one(s.a, lane);
    if constexpr (NB > 0) shift_up_one(s.b, lane);
    if constexpr (NA > 0) {
#pragma unroll
        for (int k = 0; k < NA; ++k) {
            s.a.z[k][0] += e.a.z[k][0];
            s.a.z[k][1] += e.a.z[k][1];
        }
    }
    if constexpr (NB > 0) {
#pragma unroll
        for (int k = 0; k < NB; ++k) {
            s.b.z[k][0] += e.b.z[k][0];
            s.b.z[k][1] += e.b.z[k][1];
        }
    }

    // second run from the true start state, emitting outputs
    double acc = 0.0;
#pragma unroll
    for (int i = 0; i < kChunk; ++i) {
        const int64_t j = j0 + i;
        double xa = 0.0, xb = 0.0;
        const int64_t n = Mode::kReverse ? len - 1 - j : j;
        if (j < len) m.inputs(n, in[i], xa, xb);
        double ya = 0.0, yb = 0.0;
        if constexpr (NA > 0) ya = ca.step(s.a, xa);
        if constexpr (NB > 0) yb = cb.step(s.b, xb);
        if (j < len) m.emit(row, n, ya, yb, acc, consts);
    }

    if constexpr (Mode::kAccumulates) {
        acc = wave_sum(acc);
        if (lane == 0) accum[wave] = acc;
        __syncthreads();
        if (threadIdx.x == 0) {
            double total = accum[0];
            for (int i = 1; i < kWaves; ++i) total += accum[i];
            m.finish(row, blk, total);
        }
    }
}

}  // namespace pesq
