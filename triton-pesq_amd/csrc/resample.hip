// Polyphase windowed-sinc resampler (the TritonResample operator) and its
// adjoint.
//
// torchaudio's conv form (used by the reference, triton_ops/resample.py:9-37):
//     y[l new + j] = sum_k K[j, k] x[l orig + k - width],   x = 0 outside [0, n_in)
// Only a contiguous band of taps [tap_lo[j], tap_hi[j]) of each phase is
// non-zero in float32 (the window vanishes outside |t| < lowpass width), so
// only those are evaluated: 33-34 per output at 44.1 -> 16 kHz instead of 475.
// Products are accumulated in float64.
//
// The adjoint is a gather over input samples, no atomics: input sample i is
// read by output (l, j) through tap k = i + width - l orig; for each tap k the
// phases with a non-zero K[j, k] form the range [phase_lo[k], phase_hi[k]).
#include <algorithm>
#include <cstring>
#include <vector>

#include "common.hpp"

namespace pesq {

constexpr int kResampleThreads = 256;

// The rows of one launch: rows below `split` are rows of p, the others rows
// of p2 (split = the row count for one signal; two signals of one shape, the
// reference and the degraded signal, can share a launch).
template <typename T>
struct Rows {
    T *p, *p2;
    int64_t split;
    __host__ __device__ __forceinline__ T *row(int64_t r, int64_t n) const {
        return r < split ? p + r * n : p2 + (r - split) * n;
    }
};
using InRows = Rows<const float>;
using OutRows = Rows<float>;

__global__ void __launch_bounds__(kResampleThreads)
    resample_fwd_kernel(InRows x, OutRows y, int64_t n_in,
                        int64_t n_out, const float *__restrict__ kernel,
                        const int32_t *__restrict__ tap_lo, const int32_t *__restrict__ tap_hi,
                        int64_t orig, int64_t nstep, int64_t width, int64_t wtotal,
                        int64_t blocks_per_row) {
    const int64_t row = blockIdx.x / blocks_per_row;
    const int64_t m = (blockIdx.x - row * blocks_per_row) * int64_t(blockDim.x) + threadIdx.x;
    if (m >= n_out) return;
    const int64_t l = m / nstep;
    const int64_t j = m - l * nstep;
    const float *xr = x.row(row, n_in);
    const float *kr = kernel + j * wtotal;
    const int64_t base = l * orig - width;
    const int lo = tap_lo[j], hi = tap_hi[j];
    double acc = 0.0;
    for (int k = lo; k < hi; ++k) {
        const int64_t i = base + k;
        if (i >= 0 && i < n_in) acc = fma(static_cast<double>(kr[k]), static_cast<double>(xr[i]), acc);
    }
    y.row(row, n_out)[m] = static_cast<float>(acc);
}

__global__ void __launch_bounds__(kResampleThreads)
    resample_bwd_kernel(InRows gy, OutRows gx, int64_t n_in,
                        int64_t n_out, const float *__restrict__ kernel,
                        const int32_t *__restrict__ phase_lo, const int32_t *__restrict__ phase_hi,
                        int64_t orig, int64_t nstep, int64_t width, int64_t wtotal,
                        int64_t blocks_per_row) {
    const int64_t row = blockIdx.x / blocks_per_row;
    const int64_t i = (blockIdx.x - row * blocks_per_row) * int64_t(blockDim.x) + threadIdx.x;
    if (i >= n_in) return;
    const float *gr = gy.row(row, n_out);
    const int64_t shifted = i + width;
    const int64_t l0 = shifted / orig;
    const int64_t rho = shifted - l0 * orig;
    double acc = 0.0;
    for (int64_t k = rho, l = l0; k < wtotal && l >= 0; k += orig, --l) {
        const int jlo = phase_lo[k], jhi = phase_hi[k];
        for (int j = jlo; j < jhi; ++j) {
            const int64_t m = l * nstep + j;
            if (m < n_out) {
                acc = fma(static_cast<double>(kernel[int64_t(j) * wtotal + k]),
                          static_cast<double>(gr[m]), acc);
            }
        }
    }
    gx.row(row, n_in)[i] = static_cast<float>(acc);
}

// ---------------------------------------------------------------------------
// tiled kernels: a workgroup stages the samples its outputs (inputs) read in
// LDS, the non-zero taps come from compact zero-padded tables, and every
// thread keeps kQ independent accumulators (kQ outputs 256 apart), so the
// tap loops carry no bounds checks and no dependence chain longer than the
// tap count of one output.
//
// Forward table taps[t][j] = K[j][tap_lo[j] + t] (0 past the phase's run),
// offs[j] = tap_lo[j] - width:
//     y[l nstep + j] = sum_{t < T} taps[t][j] x[l orig + offs[j] + t].
// Adjoint tables per column k < S orig (S = ceil(wtotal / orig), columns at
// or past wtotal are zero): cols[p][k] = K[col_lo[k] + p][k] for the phases
// col_lo[k] .. col_lo[k] + count - 1 whose run contains k, 0 past them:
//     gx[i] = sum_{s < S} sum_{p < P} cols[p][k_s] gy[(l0 - s) nstep + col_lo[k_s] + p],
// k_s = rho + s orig, l0 = (i + width) / orig, rho = (i + width) mod orig.
// Both sums run in the order of the untiled kernels (taps ascending; s, then
// phase ascending), zero padded terms add exact zeros.
// ---------------------------------------------------------------------------

// Staging of a row segment into LDS.  stage_row4 copies samples lo .. lo +
// span - 1 of a row of n (sample s at s + s / kPad for kPad > 0, else at s),
// zero outside the row, with 16 byte loads: thread t of a batch takes the
// four staged samples 4 (t + 256 k) .. + 3, and issues all kBatch4 loads of a
// batch before any of their LDS writes, so that a batch costs one memory round
// trip (a plain loop waits for every load before its write).  The load starts
// at the clamped sample st = clamp(lo + s, 0, n - 4) (a row of n >= 4), so it
// stays inside the row; at a row edge the lane picks its samples out of the
// loaded four by their shift from st and masks those outside the row.  No
// load depends on a condition (which would let the compiler move it under a
// branch and wait for it there), and the destination holds
// staged_floats4<kPad, kBatch4>(span) floats: span rounded up to whole
// batches.  kPad is a multiple of 4, so the four samples of a thread stay
// contiguous in the padded layout.
constexpr int kStageBatch = 8;  // staged samples per thread and batch of the tiled kernels

__host__ __device__ constexpr int64_t staged_floats(int64_t span, int pad,
                                                    int batch = kStageBatch) {
    const int64_t round = int64_t(kResampleThreads) * batch;
    const int64_t r = (span + round - 1) / round * round;
    return pad > 0 ? r + r / pad + 1 : r;
}

template <int kPad, int kBatch4>
__host__ __device__ constexpr int64_t staged_floats4(int64_t span) {
    const int64_t round = int64_t(kResampleThreads) * 4 * kBatch4;
    const int64_t r = (span + round - 1) / round * round;
    return kPad > 0 ? r + r / kPad + 1 : r;
}

template <int kPad, int kBatch4>
__device__ __forceinline__ void stage_row4(float *__restrict__ dst, const float *__restrict__ src,
                                           int64_t lo, int64_t n, int span) {
    static_assert(kPad % 4 == 0, "four samples stay contiguous");
    constexpr int kRound = kResampleThreads * 4 * kBatch4;
    if (n < 4) {  // rows of fewer than 4 samples: the plain copy
        for (int s = threadIdx.x; s < staged_floats4<0, kBatch4>(span); s += kResampleThreads) {
            const int64_t i = lo + s;
            dst[kPad > 0 ? s + s / kPad : s] = (i >= 0 && i < n) ? src[i] : 0.0f;
        }
        return;
    }
    const int span4 = (span + 3) & ~3;
    if (lo >= 0 && lo + span4 <= n) {
        // the segment lies inside the row (every workgroup but those at the
        // row ends): no clamps or masks.  Groups past the span load the
        // span's last group again (the same cache lines, no extra memory
        // traffic) and are not written.
        const float *seg = src + lo;
        for (int s0 = 0; s0 < span; s0 += kRound) {
            float q[kBatch4][4];
#pragma unroll
            for (int k = 0; k < kBatch4; ++k) {
                const int s = s0 + 4 * (k * kResampleThreads + static_cast<int>(threadIdx.x));
                __builtin_memcpy(q[k], seg + (s < span4 ? s : span4 - 4), sizeof(q[k]));
            }
#pragma unroll
            for (int k = 0; k < kBatch4; ++k) {
                const unsigned s = s0 + 4 * (k * kResampleThreads + threadIdx.x);
                if (s < unsigned(span)) {
                    float *o = dst + (kPad > 0 ? s + s / kPad : s);
#pragma unroll
                    for (int e = 0; e < 4; ++e) o[e] = q[k][e];
                }
            }
        }
        return;
    }
    for (int s0 = 0; s0 < span; s0 += kRound) {
        // all loads of the batch first, then the edge selection, then the writes
        float q[kBatch4][4];
        int64_t g0[kBatch4];
        int d[kBatch4];  // shift of the load from the first sample: 0 inside the row
#pragma unroll
        for (int k = 0; k < kBatch4; ++k) {
            g0[k] = lo + s0 + 4 * (k * kResampleThreads + static_cast<int>(threadIdx.x));
            const int64_t st = g0[k] < 0 ? 0 : (g0[k] > n - 4 ? n - 4 : g0[k]);
            d[k] = static_cast<int>(g0[k] - st);
            __builtin_memcpy(q[k], src + st, sizeof(q[k]));
        }
        float v[kBatch4][4];
#pragma unroll
        for (int k = 0; k < kBatch4; ++k) {
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const int j = e + d[k];
                const float val =
                    j <= 0 ? q[k][0] : (j == 1 ? q[k][1] : (j == 2 ? q[k][2] : q[k][3]));
                const uint32_t keep = (g0[k] + e >= 0 && g0[k] + e < n) ? 0xFFFFFFFFu : 0u;
                v[k][e] = __uint_as_float(__float_as_uint(val) & keep);
            }
        }
#pragma unroll
        for (int k = 0; k < kBatch4; ++k) {
            const unsigned s = s0 + 4 * (k * kResampleThreads + threadIdx.x);
            float *o = dst + (kPad > 0 ? s + s / kPad : s);
#pragma unroll
            for (int e = 0; e < 4; ++e) o[e] = v[k][e];
        }
    }
}

// Copy of a table of n floats into LDS; every thread issues the loads of a
// batch of 8 before their stores (indices clamped into the table, values past
// its end dropped), so that a batch costs one memory round trip instead of 8.
__device__ __forceinline__ void stage_table(float *__restrict__ dst, const float *__restrict__ src,
                                            int n) {
    constexpr int kBatch = 8;
    for (int s0 = 0; s0 < n; s0 += kResampleThreads * kBatch) {
        float v[kBatch];
#pragma unroll
        for (int b = 0; b < kBatch; ++b) {
            const int s = s0 + b * kResampleThreads + static_cast<int>(threadIdx.x);
            v[b] = src[s < n ? s : n - 1];
        }
#pragma unroll
        for (int b = 0; b < kBatch; ++b) {
            const int s = s0 + b * kResampleThreads + static_cast<int>(threadIdx.x);
            if (s < n) dst[s] = v[b];
        }
    }
}

constexpr int kTileQ = 4;
constexpr int kTileOut = kResampleThreads * kTileQ;
constexpr int kMaxSpan = 8192;   // staged samples per workgroup (32 KiB)
constexpr int kMaxTable = 8192;  // tap table floats staged in LDS (32 KiB)

// where the forward reads its taps
enum TapSource { kTapsGlobal = 0, kTapsLds = 1, kTapsUniform = 2 };

template <int kSource>
__global__ void __launch_bounds__(kResampleThreads)
    resample_fwd_tiled(InRows x, OutRows y, int64_t n_in,
                       int64_t n_out, const float *__restrict__ taps,
                       const double *__restrict__ taps64, const int32_t *__restrict__ offs,
                       int orig, int nstep, int ntaps, int off_min, int span,
                       int64_t blocks_per_row) {
    extern __shared__ float lds[];
    float *xs = lds;
    float *tl = lds + staged_floats(span, 0);
    const int64_t row = blockIdx.x / blocks_per_row;
    const int64_t m0 = (blockIdx.x - row * blocks_per_row) * kTileOut;
    const int64_t l_first = m0 / nstep;
    const int64_t in_lo = l_first * orig + off_min;
    const float *xr = x.row(row, n_in);
    stage_row4<0, kStageBatch / 4>(xs, xr, in_lo, n_in, span);
    if constexpr (kSource == kTapsLds) stage_table(tl, taps, ntaps * nstep);
    __syncthreads();
    int j[kTileQ], base[kTileQ];
    double acc[kTileQ];
#pragma unroll
    for (int q = 0; q < kTileQ; ++q) {
        const int64_t m = m0 + threadIdx.x + int64_t(kResampleThreads) * q;
        const int64_t l = m / nstep;
        j[q] = static_cast<int>(m - l * nstep);
        base[q] = static_cast<int>((l - l_first) * orig + offs[j[q]] - off_min);
        acc[q] = 0.0;
    }
    if constexpr (kSource == kTapsUniform) {
        // one phase: every lane applies the same tap, read once per wavefront
        for (int t = 0; t < ntaps; ++t) {
            const double w = taps64[t];
#pragma unroll
            for (int q = 0; q < kTileQ; ++q) {
                acc[q] = fma(w, static_cast<double>(xs[base[q] + t]), acc[q]);
            }
        }
    } else {
        const float *tt = kSource == kTapsLds ? tl : taps;
        for (int t = 0; t < ntaps; ++t) {
            const float *row_t = tt + t * nstep;
#pragma unroll
            for (int q = 0; q < kTileQ; ++q) {
                acc[q] = fma(static_cast<double>(row_t[j[q]]), static_cast<double>(xs[base[q] + t]),
                             acc[q]);
            }
        }
    }
    float *yr = y.row(row, n_out);
#pragma unroll
    for (int q = 0; q < kTileQ; ++q) {
        const int64_t m = m0 + threadIdx.x + int64_t(kResampleThreads) * q;
        if (m < n_out) yr[m] = static_cast<float>(acc[q]);
    }
}

// Phase-major kernel for rate pairs of many phases (44.1 -> 16 kHz is 441:160,
// its adjoint through the transposed bank 160:441): thread (j, h) of a
// workgroup of `groups` x nstep threads computes phase j of kP consecutive
// periods h kP .. h kP + kP - 1 of the workgroup's, with phase j's taps held
// in registers as doubles (converted once), so that a tap costs one LDS read
// of a staged sample and one FMA (the tiled kernel reads a tap and a sample
// and converts both); the samples are staged as S (double, or float
// converted per tap where the reads would cost more than the conversion).  The taps are the tiled
// kernel's zero-padded table, and each sum runs over them in ascending order
// from zero, the tiled kernel's operations, followed by exact zero terms up
// to a multiple of four taps: the same outputs for finite samples.
constexpr int kPhaseMinPhases = 64;     // fewer phases: the tiled kernel
constexpr int kPhaseMaxThreads = 512;   // threads per workgroup
constexpr int kPhasePeriods = 4;        // periods per thread
constexpr int kPhaseLds = 65536;        // bytes of staged samples a workgroup may hold

// Staging of samples lo .. lo + span - 1 of a row of n (zero outside it) as S
// (float or double), by any number of threads: four samples per thread with
// 16-byte loads, two loads per thread issued before their LDS writes.  The
// destination holds span rounded up to a multiple of 4 values.
template <typename S>
__device__ __forceinline__ void stage_row_as(S *__restrict__ dst, const float *__restrict__ src,
                                             int64_t lo, int64_t n, int span) {
    const int nt = static_cast<int>(blockDim.x), tid = static_cast<int>(threadIdx.x);
    const int span4 = (span + 3) & ~3;
    if (n >= 4 && lo >= 0 && lo + span4 <= n) {
        constexpr int kB = 2;
        const float *seg = src + lo;
        for (int s0 = 0; s0 < span; s0 += 4 * kB * nt) {
            float q[kB][4];
#pragma unroll
            for (int k = 0; k < kB; ++k) {
                const int s = s0 + 4 * (k * nt + tid);
                __builtin_memcpy(q[k], seg + (s < span4 ? s : span4 - 4), sizeof(q[k]));
            }
#pragma unroll
            for (int k = 0; k < kB; ++k) {
                const int s = s0 + 4 * (k * nt + tid);
                if (s < span) {
#pragma unroll
                    for (int e = 0; e < 4; ++e) dst[s + e] = static_cast<S>(q[k][e]);
                }
            }
        }
        return;
    }
    for (int s = tid; s < span4; s += nt) {
        const int64_t i = lo + s;
        dst[s] = (s < span && i >= 0 && i < n) ? static_cast<S>(src[i]) : S(0);
    }
}

// y[l nstep + j] = sum_{t < kTaps} taps[t][j] x[l orig + offs[j] + t] (x zero
// outside the row), the taps past ntaps zero: the tap loop is unrolled with
// no condition (a condition per tap makes the compiler wait out each tap's
// LDS reads before the next tap's), and the staged window covers kTaps.
template <int kTaps, typename S>
__global__ void __launch_bounds__(kPhaseMaxThreads)
    resample_phase_major(InRows x, OutRows y, int64_t n_in,
                         int64_t n_out, const float *__restrict__ taps,
                         const int32_t *__restrict__ offs, int orig, int nstep, int ntaps,
                         int off_min, int groups, int span, int64_t blocks_per_row) {
    extern __shared__ double lds_phase[];
    S *xs_phase = reinterpret_cast<S *>(lds_phase);
    const int64_t row = blockIdx.x / blocks_per_row;
    const int64_t blk = blockIdx.x - row * blocks_per_row;
    const int tid = static_cast<int>(threadIdx.x);
    const int h = tid / nstep, j = tid - h * nstep;
    const bool active = h < groups;
    const int jj = active ? j : 0;
    // the phase's taps and offset, requested before the staging (rows past
    // ntaps read the last row and are zeroed)
    double w[kTaps];
#pragma unroll
    for (int t = 0; t < kTaps; ++t) {
        const float v = taps[int64_t(t < ntaps ? t : ntaps - 1) * nstep + jj];
        w[t] = t < ntaps ? static_cast<double>(v) : 0.0;
    }
    const int base = offs[jj] - off_min;
    const int64_t l0 = blk * groups * kPhasePeriods;  // first period of the workgroup
    stage_row_as<S>(xs_phase, x.row(row, n_in), l0 * orig + off_min, n_in, span);
    __syncthreads();
    if (!active) return;
    double acc[kPhasePeriods];
    const S *src[kPhasePeriods];
#pragma unroll
    for (int q = 0; q < kPhasePeriods; ++q) {
        acc[q] = 0.0;
        src[q] = xs_phase + (h * kPhasePeriods + q) * orig + base;
    }
    // four taps at a time: the empty asm statements pin each group's sums
    // before the next group's reads, which keeps the compiler from hoisting
    // every LDS read to the top (that takes all 256 VGPRs and spills)
#pragma unroll
    for (int t = 0; t < kTaps; ++t) {
#pragma unroll
        for (int q = 0; q < kPhasePeriods; ++q) {
            acc[q] = fma(w[t], static_cast<double>(src[q][t]), acc[q]);
        }
        if (t % 4 == 3) {
#pragma unroll
            for (int q = 0; q < kPhasePeriods; ++q) asm volatile("" : "+v"(acc[q]));
        }
    }
    float *yr = y.row(row, n_out);
#pragma unroll
    for (int q = 0; q < kPhasePeriods; ++q) {
        const int64_t m = (l0 + h * kPhasePeriods + q) * nstep + j;
        if (m < n_out) yr[m] = static_cast<float>(acc[q]);
    }
}

// Groups of nstep threads per workgroup of resample_phase_major: the count
// whose threads fill their wavefronts best (ties: more groups); 0 when the
// kernel does not apply.
static int phase_groups(int nstep) {
    if (nstep < kPhaseMinPhases || nstep > kPhaseMaxThreads) return 0;
    int best = 0;
    double best_fill = 0.0;
    for (int g = 1; g * nstep <= kPhaseMaxThreads; ++g) {
        const int threads = (g * nstep + kWave - 1) / kWave * kWave;
        if (threads > kPhaseMaxThreads) break;
        const double fill = double(g * nstep) / threads;
        if (fill >= best_fill) {
            best_fill = fill;
            best = g;
        }
    }
    return best;
}

// Launches resample_phase_major when the pair suits it (false otherwise):
// y [rows, n_out] from x [rows, n_in] with the table taps [ntaps][nstep] and
// offsets offs[nstep] in off_min .. off_max.
static bool launch_phase_major(InRows x, OutRows y, int64_t rows, int64_t n_in,
                               int64_t n_out, const float *taps, const int32_t *offs, int orig,
                               int nstep, int ntaps, int off_min, int off_max,
                               hipStream_t stream) {
    // The samples are staged as doubles where a period reads at most nstep of
    // them (upsampling, and the adjoint of downsampling through the transposed
    // bank): the phases of a wavefront then read overlapping windows, largely
    // the same LDS words, and no conversion is left in the tap loop (c3
    // adjoint 10.5-10.8 us, 11.2-11.3 with floats).  With orig > nstep (the
    // 441:160 forward) consecutive phases read about orig / nstep samples
    // apart, and 8-byte reads per tap cost more than the tiled kernel (15.5
    // against 14.2 us at c3), so the samples stay floats, converted per tap
    // (11.0-11.4 us).
    const int groups = phase_groups(nstep);
    if (groups == 0 || ntaps < 1 || ntaps > 40) return false;
    const bool wide = orig > nstep;  // float staging
    const int ktaps = (ntaps + 3) / 4 * 4;  // the instantiation: taps rounded up to 4
    const int64_t periods = int64_t(groups) * kPhasePeriods;
    const int64_t span = (periods - 1) * orig + (off_max - off_min) + ktaps;
    const int64_t lds = (span + 3) / 4 * 4 * int64_t(wide ? sizeof(float) : sizeof(double));
    if (lds > kPhaseLds) return false;
    const int64_t bpr = cdiv(cdiv(n_out, int64_t(nstep)), periods);
    if (rows * bpr >= (int64_t(1) << 31)) return false;
    const int threads = (groups * nstep + kWave - 1) / kWave * kWave;
    const dim3 grid(static_cast<unsigned>(rows * bpr)), block(static_cast<unsigned>(threads));
#define PESQ_PHASE_MAJOR(K)                                                                      \
    case K:                                                                                       \
        if (wide) {                                                                               \
            hipLaunchKernelGGL((resample_phase_major<K, float>), grid, block, size_t(lds), stream, \
                               x, y, n_in, n_out, taps, offs, orig, nstep, ntaps, off_min, groups, \
                               static_cast<int>(span), bpr);                                      \
        } else {                                                                                  \
            hipLaunchKernelGGL((resample_phase_major<K, double>), grid, block, size_t(lds),       \
                               stream, x, y, n_in, n_out, taps, offs, orig, nstep, ntaps, off_min, \
                               groups, static_cast<int>(span), bpr);                              \
        }                                                                                         \
        return true;
    switch (ktaps) {
        PESQ_PHASE_MAJOR(4)
        PESQ_PHASE_MAJOR(8)
        PESQ_PHASE_MAJOR(12)
        PESQ_PHASE_MAJOR(16)
        PESQ_PHASE_MAJOR(20)
        PESQ_PHASE_MAJOR(24)
        PESQ_PHASE_MAJOR(28)
        PESQ_PHASE_MAJOR(32)
        PESQ_PHASE_MAJOR(36)
        PESQ_PHASE_MAJOR(40)
        default:
            return false;
    }
#undef PESQ_PHASE_MAJOR
}

// Single phase forward (new_step 1, decimation by kOrig) with a register
// window: thread u computes the kR consecutive outputs m0 + kR u + r.  With
// the taps taken in chunks t = kOrig c + d, output r reads the staged sample
// b + kOrig (r + c) + d (b = kR kOrig u: the phase's first tap is the first
// staged sample), so the rows
// X[j][d] = xs[b + kOrig j + d] form a window that slides by one row per
// chunk: every staged sample is read and converted to double once and used by
// up to kR outputs (the plain kernel reads and converts it for each of them).
// The sum of each output runs over the taps in ascending order from 0, the
// same operations as resample_fwd_tiled<kTapsUniform>.
constexpr int kWinOut = 8;  // outputs per thread
// staging batch of resample_fwd_window (float4 loads per thread): 1024
// (2 orig + 1) samples, the window of 2048 outputs and up to 1024 / orig taps
__host__ __device__ constexpr int fwd_window_batch4(int orig) { return 2 * orig + 1; }
constexpr int kMaxWindowLds = 65536;  // bytes of LDS a window kernel may stage

template <int kOrig>
__global__ void __launch_bounds__(kResampleThreads)
    resample_fwd_window(InRows x, OutRows y, int64_t n_in,
                        int64_t n_out, const double *__restrict__ taps64, int ntaps, int off_min,
                        int span, int64_t blocks_per_row) {
    constexpr int kR = kWinOut;
    constexpr int kTile = kResampleThreads * kR;
    constexpr int kStride = kR * kOrig;  // staged samples between the windows of two lanes
    extern __shared__ float lds[];
    // staged sample s at s + s / kStride: one word of padding per lane stride
    // makes the lane stride kStride + 1 words, odd, so a wavefront's reads of
    // one window row fall in distinct banks
    float *xs = lds;
    const int64_t row = blockIdx.x / blocks_per_row;
    const int64_t m0 = (blockIdx.x - row * blocks_per_row) * kTile;
    const int64_t in_lo = m0 * kOrig + off_min;
    const float *xr = x.row(row, n_in);
    stage_row4<kStride, fwd_window_batch4(kOrig)>(xs, xr, in_lo, n_in, span);
    __syncthreads();
    // staged sample kStride u + o of lane u sits at xl[o + o / kStride]; a
    // group of kR chunks advances the window by kStride samples, so the reads
    // of a group take compile time offsets from a base that moves by
    // kStride + 1 words per group
    const float *xl = xs + (kStride + 1) * static_cast<int>(threadIdx.x);
    double win[kR][kOrig];  // row j of the window in slot j mod kR
#pragma unroll
    for (int j = 0; j < kR - 1; ++j) {
#pragma unroll
        for (int d = 0; d < kOrig; ++d) {
            const int o = kOrig * j + d;
            win[j][d] = static_cast<double>(xl[o + o / kStride]);
        }
    }
    double acc[kR];
#pragma unroll
    for (int r = 0; r < kR; ++r) acc[r] = 0.0;
    // chunk g kR + cc of a group at base xg (rows g kR ...), taps tg[kOrig cc + d];
    // kTail: the last group, whose taps may end inside it (rem of them left)
    auto group = [&](const float *xg, const double *tg, auto tail, int rem) {
        constexpr bool kTail = decltype(tail)::value;
#pragma unroll
        for (int cc = 0; cc < kR; ++cc) {
            if (kTail && kOrig * cc >= rem) break;
            // row g kR + cc + kR - 1 enters the window
#pragma unroll
            for (int d = 0; d < kOrig; ++d) {
                const int o = kOrig * (cc + kR - 1) + d;
                win[(cc + kR - 1) % kR][d] = static_cast<double>(xg[o + o / kStride]);
            }
#pragma unroll
            for (int d = 0; d < kOrig; ++d) {
                if (kTail && kOrig * cc + d >= rem) break;
                const double w = tg[kOrig * cc + d];
#pragma unroll
                for (int r = 0; r < kR; ++r) acc[r] = fma(w, win[(cc + r) % kR][d], acc[r]);
            }
        }
    };
    const int full = ntaps / kStride;  // groups whose taps all exist
    const float *xg = xl;
    const double *tg = taps64;
    for (int g = 0; g < full; ++g, xg += kStride + 1, tg += kStride) {
        group(xg, tg, std::false_type{}, kStride);
    }
    if (ntaps > full * kStride) group(xg, tg, std::true_type{}, ntaps - full * kStride);
    float *yr = y.row(row, n_out);
    float res[kR];
#pragma unroll
    for (int r = 0; r < kR; ++r) res[r] = static_cast<float>(acc[r]);
    const int64_t m = m0 + int64_t(kR) * threadIdx.x;
    if (m0 + kTile <= n_out) {
        __builtin_memcpy(yr + m, res, sizeof(res));  // 16 byte stores
    } else {
#pragma unroll
        for (int r = 0; r < kR; ++r) {
            if (m + r < n_out) yr[m + r] = res[r];
        }
    }
}

// staged samples of resample_fwd_window (the last window row read ends at
// orig (256 kR + nchunk - 1)), and its LDS bytes with the padding
static int64_t window_span(int orig, int ntaps) {
    const int64_t nchunk = (ntaps + orig - 1) / orig;
    return int64_t(orig) * (int64_t(kResampleThreads) * kWinOut + nchunk - 1);
}
static int64_t window_lds(int64_t span, int orig) {
    int64_t f = 0;
    switch (orig) {
        case 2: f = staged_floats4<kWinOut * 2, fwd_window_batch4(2)>(span); break;
        case 3: f = staged_floats4<kWinOut * 3, fwd_window_batch4(3)>(span); break;
        case 4: f = staged_floats4<kWinOut * 4, fwd_window_batch4(4)>(span); break;
        case 6: f = staged_floats4<kWinOut * 6, fwd_window_batch4(6)>(span); break;
        default: f = int64_t(1) << 40;  // no window kernel
    }
    return f * int64_t(sizeof(float));
}

// Adjoint of a single phase rate pair (new_step 1, integer decimation):
// thread u of the workgroup takes the orig consecutive inputs
// i = i0 + orig (u + 256 q) + c; input c of every thread uses the taps
// row[rho_c + s orig], rho_c = (c + width) mod orig, the same in every lane,
// read as float64 scalars.  The outputs go through LDS to be written with
// unit stride.
constexpr int kUniQ = 2;

__global__ void __launch_bounds__(kResampleThreads)
    resample_bwd_uniform(InRows gy, OutRows gx, int64_t n_in,
                         int64_t n_out, const double *__restrict__ row, int orig, int width,
                         int sweeps, int span, int64_t blocks_per_row) {
    extern __shared__ float lds[];
    float *gs = lds;
    float *out = lds + staged_floats(span, 0);
    const int per_block = kResampleThreads * kUniQ * orig;
    const int64_t row_id = blockIdx.x / blocks_per_row;
    const int64_t i0 = (blockIdx.x - row_id * blocks_per_row) * per_block;
    const int64_t l_lo = (i0 + width) / orig - (sweeps - 1);
    const float *gr = gy.row(row_id, n_out);
    stage_row4<0, kStageBatch / 4>(gs, gr, l_lo, n_out, span);
    __syncthreads();
    for (int c = 0; c < orig; ++c) {
        const int rho = (c + width) % orig;
        // l0 - l_lo of input u = 0 of this c; the lanes add u
        const int lrel0 = static_cast<int>((i0 + c + width) / orig - l_lo);
        double acc[kUniQ];
#pragma unroll
        for (int q = 0; q < kUniQ; ++q) acc[q] = 0.0;
        for (int sw = 0; sw < sweeps; ++sw) {
            const double w = row[rho + sw * orig];
#pragma unroll
            for (int q = 0; q < kUniQ; ++q) {
                const int u = threadIdx.x + kResampleThreads * q;
                acc[q] = fma(w, static_cast<double>(gs[lrel0 + u - sw]), acc[q]);
            }
        }
#pragma unroll
        for (int q = 0; q < kUniQ; ++q) {
            const int u = threadIdx.x + kResampleThreads * q;
            out[u * orig + c] = static_cast<float>(acc[q]);
        }
    }
    __syncthreads();
    float *gxr = gx.row(row_id, n_in);
    for (int s = threadIdx.x; s < per_block; s += kResampleThreads) {
        if (i0 + s < n_in) gxr[i0 + s] = out[s];
    }
}

// Adjoint of a single phase rate pair (new_step 1, decimation by kOrig) with
// a register window.  Input i with i + width = kOrig l + rho receives
//     gx[i] = sum_{s < sweeps} row[rho + kOrig s] gy[l - s].
// Thread u takes the kV consecutive l = l_u + v (v < kV) and all kOrig phases
// of each: the kV kOrig consecutive inputs from kOrig l_u - width.  They read
// gy[l_u + v - s], a window of kV values that slides by one per step s: each
// staged gy sample is converted to double once and feeds kV kOrig sums.  The
// sums run over s in ascending order from 0, as in resample_bwd_uniform; the
// results go through LDS to be written with unit stride.
// output positions l per thread: odd, so that the lane strides of the
// staged gradient (kWinIn words) and of the results (kWinIn orig words) are
// odd and a wavefront's LDS accesses fall in distinct banks without padding
constexpr int kWinIn = 7;
constexpr int kBwdWindowBatch4 = 2;  // staging: float4 loads per thread, 2048 samples

template <int kOrig>
__global__ void __launch_bounds__(kResampleThreads)
    resample_bwd_window(InRows gy, OutRows gx, int64_t n_in,
                        int64_t n_out, const double *__restrict__ row, int width, int sweeps,
                        int64_t l_min, int span, int64_t blocks_per_row) {
    constexpr int kV = kWinIn;
    constexpr int kPerBlock = kResampleThreads * kV;  // l per workgroup
    constexpr int kOut = kV * kOrig;                  // inputs per thread
    extern __shared__ float lds[];
    float *gs = lds;                                                // gy[l_b - sweeps + 1 + s]
    float *out = lds + staged_floats4<0, kBwdWindowBatch4>(span);  // the block's inputs
    const int64_t row_id = blockIdx.x / blocks_per_row;
    const int64_t l_b = l_min + (blockIdx.x - row_id * blocks_per_row) * kPerBlock;
    const int64_t g_lo = l_b - sweeps + 1;
    const float *gr = gy.row(row_id, n_out);
    stage_row4<0, kBwdWindowBatch4>(gs, gr, g_lo, n_out, span);
    __syncthreads();
    // gy[l_u + p] is staged sample kV u + sweeps - 1 + p, p = v - s
    const float *gl = gs + kV * static_cast<int>(threadIdx.x) + sweeps - 1;
    auto grad = [&](int p) { return static_cast<double>(gl[p]); };
    double win[kV];  // gy[l_u + p] in slot p mod kV
#pragma unroll
    for (int p = 1; p < kV; ++p) win[p] = grad(p);
    double acc[kV][kOrig];
#pragma unroll
    for (int v = 0; v < kV; ++v) {
#pragma unroll
        for (int r = 0; r < kOrig; ++r) acc[v][r] = 0.0;
    }
    for (int s0 = 0; s0 < sweeps; s0 += kV) {
#pragma unroll
        for (int ss = 0; ss < kV; ++ss) {
            const int sw = s0 + ss;
            if (sw >= sweeps) break;
            // p = -sw enters the window (v = 0), in the slot of p = kV - sw
            win[(kV - ss) % kV] = grad(-sw);
#pragma unroll
            for (int r = 0; r < kOrig; ++r) {
                const double w = row[r + kOrig * sw];
#pragma unroll
                for (int v = 0; v < kV; ++v) acc[v][r] = fma(w, win[(v - ss + kV) % kV], acc[v][r]);
            }
        }
    }
    float *ol = out + kOut * static_cast<int>(threadIdx.x);
#pragma unroll
    for (int v = 0; v < kV; ++v) {
#pragma unroll
        for (int r = 0; r < kOrig; ++r) ol[v * kOrig + r] = static_cast<float>(acc[v][r]);
    }
    __syncthreads();
    // input of result k: kOrig l_b - width + k
    const int64_t i_b = kOrig * l_b - width;
    float *gxr = gx.row(row_id, n_in);
    constexpr int kResults = kPerBlock * kOrig;
    static_assert(kResults % 4 == 0, "results in groups of four");
    if (i_b >= 0 && i_b + kResults <= n_in) {
        // inside the row: 16 byte LDS reads (the result region starts at a
        // multiple of 4 floats) and 16 byte global stores
        for (int g = threadIdx.x; g < kResults / 4; g += kResampleThreads) {
            float v[4];
            __builtin_memcpy(v, out + 4 * g, sizeof(v));
            __builtin_memcpy(gxr + i_b + 4 * g, v, sizeof(v));
        }
    } else {
        for (int k = threadIdx.x; k < kResults; k += kResampleThreads) {
            const int64_t i = i_b + k;
            if (i >= 0 && i < n_in) gxr[i] = out[k];
        }
    }
}

// staged gy samples of resample_bwd_window and its LDS bytes
static int64_t bwd_window_span(int sweeps) {
    return int64_t(kResampleThreads) * kWinIn + sweeps - 1;
}
static int64_t bwd_window_lds(int64_t span, int orig) {
    const int64_t results = int64_t(kResampleThreads) * kWinIn * orig;
    return (staged_floats4<0, kBwdWindowBatch4>(span) + results) * int64_t(sizeof(float));
}

template <bool kLds>
__global__ void __launch_bounds__(kResampleThreads)
    resample_bwd_tiled(InRows gy, OutRows gx, int64_t n_in,
                       int64_t n_out, const float *__restrict__ cols,
                       const int32_t *__restrict__ col_lo, int orig, int nstep, int width,
                       int nphases, int sweeps, int ncols, int span, int64_t blocks_per_row) {
    extern __shared__ float lds[];
    float *gs = lds;
    float *cl = lds + staged_floats(span, 0);
    int32_t *clo = reinterpret_cast<int32_t *>(cl + nphases * ncols);
    const int64_t row = blockIdx.x / blocks_per_row;
    const int64_t i0 = (blockIdx.x - row * blocks_per_row) * kTileOut;
    const int64_t l_lo = (i0 + width) / orig - (sweeps - 1);
    const int64_t m_lo = l_lo * nstep;  // may be negative: those outputs read as zero
    const float *gr = gy.row(row, n_out);
    stage_row4<0, kStageBatch / 4>(gs, gr, m_lo, n_out, span);
    if constexpr (kLds) {
        for (int s = threadIdx.x; s < nphases * ncols; s += kResampleThreads) cl[s] = cols[s];
        for (int s = threadIdx.x; s < ncols; s += kResampleThreads) clo[s] = col_lo[s];
    }
    __syncthreads();
    const float *cc = kLds ? cl : cols;
    const int32_t *cq = kLds ? clo : col_lo;
    float *gxr = gx.row(row, n_in);
#pragma unroll
    for (int q = 0; q < kTileQ; ++q) {
        const int64_t i = i0 + threadIdx.x + int64_t(kResampleThreads) * q;
        const int64_t sh = i + width;
        const int64_t l0 = sh / orig;
        const int rho = static_cast<int>(sh - l0 * orig);
        const int lrel = static_cast<int>(l0 - l_lo);
        double acc = 0.0;
        for (int sw = 0; sw < sweeps; ++sw) {
            const int k = rho + sw * orig;
            const int mb = (lrel - sw) * nstep + cq[k];
            for (int p = 0; p < nphases; ++p) {
                acc = fma(static_cast<double>(cc[p * ncols + k]), static_cast<double>(gs[mb + p]), acc);
            }
        }
        if (i < n_in) gxr[i] = static_cast<float>(acc);
    }
}

}  // namespace pesq

using namespace pesq;

static int check_resample(int64_t rows, int64_t n_in, int64_t n_out, int64_t orig, int64_t nstep,
                          int64_t width, int64_t wtotal) {
    PESQ_CHECK_ARG(rows >= 0 && n_in >= 0 && n_out >= 0, "invalid sizes");
    PESQ_CHECK_ARG(orig > 0 && nstep > 0 && width >= 0 && wtotal > 0, "invalid resampling steps");
    PESQ_CHECK_ARG(wtotal == 2 * width + orig, "width_total must be 2 width + orig_step");
    return PESQ_OK;
}

extern "C" int pesq_resample_forward(const float *x, float *y, int64_t rows, int64_t n_in,
                                     int64_t n_out, const float *kernel, const int32_t *tap_lo,
                                     const int32_t *tap_hi, int64_t orig_step, int64_t new_step,
                                     int64_t width, int64_t width_total, hipStream_t stream) {
    if (int st = check_resample(rows, n_in, n_out, orig_step, new_step, width, width_total)) return st;
    if (rows == 0 || n_out == 0) return PESQ_OK;
    PESQ_CHECK_ARG(x && y && kernel && tap_lo && tap_hi, "null pointer argument");
    const int64_t bpr = cdiv(n_out, kResampleThreads);
    PESQ_CHECK_ARG(rows * bpr < (int64_t(1) << 31), "too many rows x blocks for one launch");
    hipLaunchKernelGGL(resample_fwd_kernel, dim3(static_cast<unsigned>(rows * bpr)),
                       dim3(kResampleThreads), 0, stream, InRows{x, x, rows}, OutRows{y, y, rows},
                       n_in, n_out, kernel, tap_lo, tap_hi, orig_step, new_step, width,
                       width_total, bpr);
    PESQ_CHECK_LAUNCH("resample forward");
    return PESQ_OK;
}

extern "C" int pesq_resample_backward(const float *grad_y, float *grad_x, int64_t rows,
                                      int64_t n_in, int64_t n_out, const float *kernel,
                                      const int32_t *phase_lo, const int32_t *phase_hi,
                                      int64_t orig_step, int64_t new_step, int64_t width,
                                      int64_t width_total, hipStream_t stream) {
    if (int st = check_resample(rows, n_in, n_out, orig_step, new_step, width, width_total)) return st;
    if (rows == 0 || n_in == 0) return PESQ_OK;
    PESQ_CHECK_ARG(grad_y && grad_x && kernel && phase_lo && phase_hi, "null pointer argument");
    const int64_t bpr = cdiv(n_in, kResampleThreads);
    PESQ_CHECK_ARG(rows * bpr < (int64_t(1) << 31), "too many rows x blocks for one launch");
    hipLaunchKernelGGL(resample_bwd_kernel, dim3(static_cast<unsigned>(rows * bpr)),
                       dim3(kResampleThreads), 0, stream, InRows{grad_y, grad_y, rows},
                       OutRows{grad_x, grad_x, rows}, n_in, n_out, kernel, phase_lo, phase_hi,
                       orig_step, new_step, width, width_total, bpr);
    PESQ_CHECK_LAUNCH("resample backward");
    return PESQ_OK;
}

static int64_t align256(int64_t v) { return (v + 255) / 256 * 256; }

extern "C" int pesq_resample_plan(const float *kernel, const int32_t *tap_lo,
                                  const int32_t *tap_hi, int64_t orig_step, int64_t new_step,
                                  int64_t width, int64_t width_total,
                                  pesq_resample_plan_info *info, void *plan) {
    PESQ_CHECK_ARG(kernel && tap_lo && tap_hi && info, "null argument");
    if (int st = check_resample(0, 0, 0, orig_step, new_step, width, width_total)) return st;
    PESQ_CHECK_ARG(orig_step < (1 << 20) && new_step < (1 << 20) && width_total < (1 << 22),
                   "resampling steps too large");
    const int orig = static_cast<int>(orig_step), nstep = static_cast<int>(new_step);
    const int wtotal = static_cast<int>(width_total);
    pesq_resample_plan_info r{};
    r.orig_step = orig;
    r.new_step = nstep;
    r.width = static_cast<int>(width);
    r.width_total = wtotal;
    int taps = 1, off_min = 1 << 30, off_max = -(1 << 30);
    for (int j = 0; j < nstep; ++j) {
        PESQ_CHECK_ARG(tap_lo[j] >= 0 && tap_lo[j] <= tap_hi[j] && tap_hi[j] <= wtotal,
                       "phase %d has an invalid tap range [%d, %d)", j, tap_lo[j], tap_hi[j]);
        taps = std::max(taps, tap_hi[j] - tap_lo[j]);
        off_min = std::min(off_min, tap_lo[j] - r.width);
        off_max = std::max(off_max, tap_lo[j] - r.width);
    }
    const int sweeps = (wtotal + orig - 1) / orig;
    const int ncols = sweeps * orig;
    // phases per column: contiguous because the runs move monotonically with j
    std::vector<int32_t> col_lo(ncols, 0), col_n(ncols, 0);
    int phases = 1;
    for (int k = 0; k < wtotal; ++k) {
        int first = -1, last = -1;
        for (int j = 0; j < nstep; ++j) {
            if (tap_lo[j] <= k && k < tap_hi[j]) {
                if (first < 0) first = j;
                PESQ_CHECK_ARG(last < 0 || last == j - 1,
                               "the phases of tap column %d are not contiguous", k);
                last = j;
            }
        }
        if (first >= 0) {
            col_lo[k] = first;
            col_n[k] = last - first + 1;
            phases = std::max(phases, col_n[k]);
        }
    }
    r.taps = taps;
    r.off_min = off_min;
    r.off_max = off_max;
    r.phases = phases;
    r.sweeps = sweeps;
    r.columns = ncols;
    // staged floats per workgroup (worst case over the workgroups)
    const int64_t fwd_periods = (kTileOut - 1) / nstep + 1;
    const int64_t fwd_span = fwd_periods * orig + (off_max - off_min) + taps;
    const int64_t bwd_periods = (kTileOut - 1 + orig - 1) / orig + 1 + sweeps;
    int64_t bwd_span = bwd_periods * nstep + phases;
    if (nstep == 1) {
        // resample_bwd_uniform: gy samples, then the block's outputs
        bwd_span = int64_t(kResampleThreads) * kUniQ + sweeps + 1;
        if (bwd_span + int64_t(kResampleThreads) * kUniQ * orig > kMaxSpan) bwd_span = kMaxSpan + 1;
    }
    r.fwd_span = fwd_span <= kMaxSpan ? static_cast<int32_t>(fwd_span) : 0;
    r.bwd_span = bwd_span <= kMaxSpan ? static_cast<int32_t>(bwd_span) : 0;
    // The adjoint as a resampler from new_step to orig_step: input i = l orig + j
    // (i + width = (l + carry) orig + rho, carry and rho from j) receives the
    // outputs m = (l + carry) nstep + m_rel over the tap columns k = rho + s orig
    // and their phases, m_rel = col_lo[k] + p - s nstep: one contiguous run of
    // outputs per j (runs of different sweeps do not overlap, and gaps between
    // them get zero taps), starting at adj_offs[j] = carry nstep + min m_rel.
    std::vector<int32_t> adj_lo(orig, 0), adj_n(orig, 0);
    int adj_taps = 1, adj_off_min = 1 << 30, adj_off_max = -(1 << 30);
    if (nstep > 1) {
        for (int j = 0; j < orig; ++j) {
            const int rho = (j + r.width) % orig, carry = (j + r.width) / orig;
            int lo = 1 << 30, hi = -(1 << 30);
            for (int s = 0; s < sweeps; ++s) {
                const int k = rho + s * orig;
                if (k >= wtotal || col_n[k] == 0) continue;
                lo = std::min(lo, col_lo[k] - s * nstep);
                hi = std::max(hi, col_lo[k] + col_n[k] - 1 - s * nstep);
            }
            if (hi < lo) lo = hi = 0;  // no tap reads this input: one zero tap
            adj_lo[j] = carry * nstep + lo;
            adj_n[j] = hi - lo + 1;
            adj_taps = std::max(adj_taps, adj_n[j]);
            adj_off_min = std::min(adj_off_min, adj_lo[j]);
            adj_off_max = std::max(adj_off_max, adj_lo[j]);
        }
        const int64_t adj_periods = (kTileOut - 1) / orig + 1;
        const int64_t adj_span = adj_periods * nstep + (adj_off_max - adj_off_min) + adj_taps;
        r.adj_taps = adj_taps;
        r.adj_off_min = adj_off_min;
        r.adj_off_max = adj_off_max;
        r.adj_span = adj_span <= kMaxSpan && int64_t(adj_taps) * orig <= kMaxTable
                         ? static_cast<int32_t>(adj_span)
                         : 0;
    }
    r.off_offs = align256(int64_t(taps) * nstep * sizeof(float));
    r.off_cols = r.off_offs + align256(int64_t(nstep) * sizeof(int32_t));
    r.off_col_lo = r.off_cols + align256(int64_t(phases) * ncols * sizeof(float));
    r.off_taps64 = r.off_col_lo + align256(int64_t(ncols) * sizeof(int32_t));
    r.off_row64 = r.off_taps64 + align256(int64_t(taps) * sizeof(double));
    r.off_adj_taps = r.off_row64 + align256(int64_t(ncols) * sizeof(double));
    r.off_adj_offs = r.off_adj_taps + align256(int64_t(r.adj_taps) * orig * sizeof(float));
    r.bytes = r.off_adj_offs + align256(int64_t(orig) * sizeof(int32_t));
    *info = r;
    if (plan == nullptr) return PESQ_OK;

    unsigned char *base = static_cast<unsigned char *>(plan);
    std::memset(base, 0, size_t(r.bytes));
    float *tt = reinterpret_cast<float *>(base);
    int32_t *offs = reinterpret_cast<int32_t *>(base + r.off_offs);
    float *cols = reinterpret_cast<float *>(base + r.off_cols);
    int32_t *clo = reinterpret_cast<int32_t *>(base + r.off_col_lo);
    double *t64 = reinterpret_cast<double *>(base + r.off_taps64);
    double *row64 = reinterpret_cast<double *>(base + r.off_row64);
    for (int t = 0; t < tap_hi[0] - tap_lo[0]; ++t) t64[t] = kernel[tap_lo[0] + t];  // phase 0
    for (int k = tap_lo[0]; k < tap_hi[0]; ++k) row64[k] = kernel[k];  // zero elsewhere
    for (int j = 0; j < nstep; ++j) {
        offs[j] = tap_lo[j] - r.width;
        for (int t = 0; t < tap_hi[j] - tap_lo[j]; ++t) {
            tt[int64_t(t) * nstep + j] = kernel[int64_t(j) * wtotal + tap_lo[j] + t];
        }
    }
    for (int k = 0; k < ncols; ++k) {
        clo[k] = col_lo[k];
        for (int p = 0; p < col_n[k]; ++p) {
            cols[int64_t(p) * ncols + k] = kernel[int64_t(col_lo[k] + p) * wtotal + k];
        }
    }
    if (r.adj_taps > 0) {
        float *adj = reinterpret_cast<float *>(base + r.off_adj_taps);
        int32_t *aoffs = reinterpret_cast<int32_t *>(base + r.off_adj_offs);
        for (int j = 0; j < orig; ++j) {
            aoffs[j] = adj_lo[j];
            const int rho = (j + r.width) % orig, carry = (j + r.width) / orig;
            for (int s = 0; s < sweeps; ++s) {
                const int k = rho + s * orig;
                if (k >= wtotal) continue;
                for (int p = 0; p < col_n[k]; ++p) {
                    const int t = carry * nstep + col_lo[k] + p - s * nstep - adj_lo[j];
                    adj[int64_t(t) * orig + j] = kernel[int64_t(col_lo[k] + p) * wtotal + k];
                }
            }
        }
    }
    return PESQ_OK;
}

// y rows from x rows (rows in all) with the plan's kernels
static int plan_forward(InRows x, OutRows y, int64_t rows, int64_t n_in, int64_t n_out,
                        const pesq_resample_plan_info *info, const void *plan,
                        hipStream_t stream) {
    PESQ_CHECK_ARG(info != nullptr, "null plan info");
    const pesq_resample_plan_info &r = *info;
    if (int st = check_resample(rows, n_in, n_out, r.orig_step, r.new_step, r.width, r.width_total)) {
        return st;
    }
    PESQ_CHECK_ARG(r.fwd_span > 0, "this rate pair has no tiled forward (window too wide)");
    if (rows == 0 || n_out == 0) return PESQ_OK;
    PESQ_CHECK_ARG(x.p && x.p2 && y.p && y.p2 && plan, "null pointer argument");
    // the base index of an output inside the staged window fits int32
    PESQ_CHECK_ARG(n_in < (int64_t(1) << 31) && n_out < (int64_t(1) << 31), "signal too long");
    const int64_t bpr = cdiv(n_out, kTileOut);
    PESQ_CHECK_ARG(rows * bpr < (int64_t(1) << 31), "too many rows x blocks for one launch");
    const unsigned char *base = static_cast<const unsigned char *>(plan);
    const float *taps = reinterpret_cast<const float *>(base);
    const double *taps64 = reinterpret_cast<const double *>(base + r.off_taps64);
    const int32_t *offs = reinterpret_cast<const int32_t *>(base + r.off_offs);
    if (r.new_step == 1) {
        // decimation by 2, 3, 4 or 6 (32, 48, 64, 96 kHz to 16 kHz): the register window
        const int64_t wspan = window_span(r.orig_step, r.taps);
        const int64_t wbpr = cdiv(n_out, int64_t(kResampleThreads) * kWinOut);
        const dim3 wgrid(static_cast<unsigned>(rows * wbpr)), wblock(kResampleThreads);
        const size_t wbytes = size_t(window_lds(wspan, r.orig_step));
        bool launched = wbytes <= size_t(kMaxWindowLds);
        if (launched) {
            switch (r.orig_step) {
                case 2:
                    hipLaunchKernelGGL(resample_fwd_window<2>, wgrid, wblock, wbytes, stream, x, y,
                                       n_in, n_out, taps64, r.taps, r.off_min,
                                       static_cast<int>(wspan), wbpr);
                    break;
                case 3:
                    hipLaunchKernelGGL(resample_fwd_window<3>, wgrid, wblock, wbytes, stream, x, y,
                                       n_in, n_out, taps64, r.taps, r.off_min,
                                       static_cast<int>(wspan), wbpr);
                    break;
                case 4:
                    hipLaunchKernelGGL(resample_fwd_window<4>, wgrid, wblock, wbytes, stream, x, y,
                                       n_in, n_out, taps64, r.taps, r.off_min,
                                       static_cast<int>(wspan), wbpr);
                    break;
                case 6:
                    hipLaunchKernelGGL(resample_fwd_window<6>, wgrid, wblock, wbytes, stream, x, y,
                                       n_in, n_out, taps64, r.taps, r.off_min,
                                       static_cast<int>(wspan), wbpr);
                    break;
                default:
                    launched = false;
            }
        }
        if (launched) {
            PESQ_CHECK_LAUNCH("resample forward (window)");
            return PESQ_OK;
        }
    }
    if (launch_phase_major(x, y, rows, n_in, n_out, taps, offs, r.orig_step, r.new_step, r.taps,
                           r.off_min, r.off_max, stream)) {
        PESQ_CHECK_LAUNCH("resample forward (phase major)");
        return PESQ_OK;
    }
    const dim3 grid(static_cast<unsigned>(rows * bpr)), block(kResampleThreads);
    const size_t span_bytes = size_t(staged_floats(r.fwd_span, 0)) * sizeof(float);
    if (r.new_step == 1) {
        hipLaunchKernelGGL(resample_fwd_tiled<kTapsUniform>, grid, block, span_bytes, stream, x,
                           y, n_in, n_out, taps, taps64, offs, r.orig_step, r.new_step, r.taps,
                           r.off_min, r.fwd_span, bpr);
    } else if (int64_t(r.taps) * r.new_step <= kMaxTable) {
        const size_t table = size_t(r.taps) * r.new_step * sizeof(float);
        hipLaunchKernelGGL(resample_fwd_tiled<kTapsLds>, grid, block, span_bytes + table, stream,
                           x, y, n_in, n_out, taps, taps64, offs, r.orig_step, r.new_step, r.taps,
                           r.off_min, r.fwd_span, bpr);
    } else {
        hipLaunchKernelGGL(resample_fwd_tiled<kTapsGlobal>, grid, block, span_bytes, stream, x,
                           y, n_in, n_out, taps, taps64, offs, r.orig_step, r.new_step, r.taps,
                           r.off_min, r.fwd_span, bpr);
    }
    PESQ_CHECK_LAUNCH("resample forward (tiled)");
    return PESQ_OK;
}

// grad_x rows from grad_y rows (rows in all) with the plan's kernels
static int plan_backward(InRows grad_y, OutRows grad_x, int64_t rows, int64_t n_in,
                         int64_t n_out, const pesq_resample_plan_info *info, const void *plan,
                         hipStream_t stream) {
    PESQ_CHECK_ARG(info != nullptr, "null plan info");
    const pesq_resample_plan_info &r = *info;
    if (int st = check_resample(rows, n_in, n_out, r.orig_step, r.new_step, r.width, r.width_total)) {
        return st;
    }
    PESQ_CHECK_ARG(r.bwd_span > 0, "this rate pair has no tiled adjoint (window too wide)");
    if (rows == 0 || n_in == 0) return PESQ_OK;
    PESQ_CHECK_ARG(grad_y.p && grad_y.p2 && grad_x.p && grad_x.p2 && plan,
                   "null pointer argument");
    PESQ_CHECK_ARG(n_in < (int64_t(1) << 31) && n_out < (int64_t(1) << 31), "signal too long");
    const int64_t bpr = cdiv(n_in, kTileOut);
    PESQ_CHECK_ARG(rows * bpr < (int64_t(1) << 31), "too many rows x blocks for one launch");
    const unsigned char *base = static_cast<const unsigned char *>(plan);
    if (r.new_step == 1) {
        // decimation by 2, 3, 4 or 6: the register window
        const int64_t wspan = bwd_window_span(r.sweeps);
        const int64_t wlds = bwd_window_lds(wspan, r.orig_step);
        const int64_t l_min = r.width / r.orig_step;
        const int64_t l_max = (n_in - 1 + r.width) / r.orig_step;
        const int64_t wnb = cdiv(l_max - l_min + 1, int64_t(kResampleThreads) * kWinIn);
        const double *row = reinterpret_cast<const double *>(base + r.off_row64);
        const dim3 wgrid(static_cast<unsigned>(rows * wnb)), wblock(kResampleThreads);
        bool launched = wlds <= kMaxWindowLds && rows * wnb < (int64_t(1) << 31);
        if (launched) {
            switch (r.orig_step) {
                case 2:
                    hipLaunchKernelGGL(resample_bwd_window<2>, wgrid, wblock, size_t(wlds), stream,
                                       grad_y, grad_x, n_in, n_out, row, r.width, r.sweeps, l_min,
                                       static_cast<int>(wspan), wnb);
                    break;
                case 3:
                    hipLaunchKernelGGL(resample_bwd_window<3>, wgrid, wblock, size_t(wlds), stream,
                                       grad_y, grad_x, n_in, n_out, row, r.width, r.sweeps, l_min,
                                       static_cast<int>(wspan), wnb);
                    break;
                case 4:
                    hipLaunchKernelGGL(resample_bwd_window<4>, wgrid, wblock, size_t(wlds), stream,
                                       grad_y, grad_x, n_in, n_out, row, r.width, r.sweeps, l_min,
                                       static_cast<int>(wspan), wnb);
                    break;
                case 6:
                    hipLaunchKernelGGL(resample_bwd_window<6>, wgrid, wblock, size_t(wlds), stream,
                                       grad_y, grad_x, n_in, n_out, row, r.width, r.sweeps, l_min,
                                       static_cast<int>(wspan), wnb);
                    break;
                default:
                    launched = false;
            }
        }
        if (launched) {
            PESQ_CHECK_LAUNCH("resample backward (window)");
            return PESQ_OK;
        }
        const int64_t per_block = int64_t(kResampleThreads) * kUniQ * r.orig_step;
        const int64_t nb = cdiv(n_in, per_block);
        PESQ_CHECK_ARG(rows * nb < (int64_t(1) << 31), "too many rows x blocks for one launch");
        const size_t lds = size_t(staged_floats(r.bwd_span, 0) + per_block) * sizeof(float);
        hipLaunchKernelGGL(resample_bwd_uniform, dim3(static_cast<unsigned>(rows * nb)),
                           dim3(kResampleThreads), lds, stream, grad_y, grad_x, n_in, n_out,
                           reinterpret_cast<const double *>(base + r.off_row64), r.orig_step,
                           r.width, r.sweeps, r.bwd_span, nb);
        PESQ_CHECK_LAUNCH("resample backward (uniform)");
        return PESQ_OK;
    }
    if (r.adj_span > 0) {
        // the transposed bank: the forward's tiled kernel from new_step to orig_step
        const float *adj = reinterpret_cast<const float *>(base + r.off_adj_taps);
        const int32_t *aoffs = reinterpret_cast<const int32_t *>(base + r.off_adj_offs);
        if (launch_phase_major(grad_y, grad_x, rows, n_out, n_in, adj, aoffs, r.new_step,
                               r.orig_step, r.adj_taps, r.adj_off_min, r.adj_off_max, stream)) {
            PESQ_CHECK_LAUNCH("resample backward (phase major)");
            return PESQ_OK;
        }
        const int64_t table = int64_t(r.adj_taps) * r.orig_step;
        const size_t lds = size_t(staged_floats(r.adj_span, 0) + table) * sizeof(float);
        hipLaunchKernelGGL(resample_fwd_tiled<kTapsLds>, dim3(static_cast<unsigned>(rows * bpr)),
                           dim3(kResampleThreads), lds, stream, grad_y, grad_x, n_out, n_in, adj,
                           nullptr, aoffs, r.new_step, r.orig_step, r.adj_taps, r.adj_off_min,
                           r.adj_span, bpr);
        PESQ_CHECK_LAUNCH("resample backward (transposed bank)");
        return PESQ_OK;
    }
    const float *cols = reinterpret_cast<const float *>(base + r.off_cols);
    const int32_t *col_lo = reinterpret_cast<const int32_t *>(base + r.off_col_lo);
    const dim3 grid(static_cast<unsigned>(rows * bpr)), block(kResampleThreads);
    const size_t span_bytes = size_t(staged_floats(r.bwd_span, 0)) * sizeof(float);
    const int64_t table = (int64_t(r.phases) + 1) * r.columns;
    if (table <= kMaxTable) {
        hipLaunchKernelGGL(resample_bwd_tiled<true>, grid, block,
                           span_bytes + size_t(table) * sizeof(float), stream, grad_y, grad_x,
                           n_in, n_out, cols, col_lo, r.orig_step, r.new_step, r.width, r.phases,
                           r.sweeps, r.columns, r.bwd_span, bpr);
    } else {
        hipLaunchKernelGGL(resample_bwd_tiled<false>, grid, block, span_bytes, stream, grad_y,
                           grad_x, n_in, n_out, cols, col_lo, r.orig_step, r.new_step, r.width,
                           r.phases, r.sweeps, r.columns, r.bwd_span, bpr);
    }
    PESQ_CHECK_LAUNCH("resample backward (tiled)");
    return PESQ_OK;
}

extern "C" int pesq_resample_plan_forward(const float *x, float *y, int64_t rows, int64_t n_in,
                                          int64_t n_out, const pesq_resample_plan_info *info,
                                          const void *plan, hipStream_t stream) {
    return plan_forward(InRows{x, x, rows}, OutRows{y, y, rows}, rows, n_in, n_out, info, plan,
                        stream);
}

extern "C" int pesq_resample_plan_forward_pair(const float *x0, float *y0, const float *x1,
                                               float *y1, int64_t rows, int64_t n_in,
                                               int64_t n_out, const pesq_resample_plan_info *info,
                                               const void *plan, hipStream_t stream) {
    PESQ_CHECK_ARG(rows >= 0 && rows < (int64_t(1) << 40), "invalid row count %lld",
                   (long long)rows);
    return plan_forward(InRows{x0, x1, rows}, OutRows{y0, y1, rows}, 2 * rows, n_in, n_out, info,
                        plan, stream);
}

extern "C" int pesq_resample_plan_backward(const float *grad_y, float *grad_x, int64_t rows,
                                           int64_t n_in, int64_t n_out,
                                           const pesq_resample_plan_info *info, const void *plan,
                                           hipStream_t stream) {
    return plan_backward(InRows{grad_y, grad_y, rows}, OutRows{grad_x, grad_x, rows}, rows, n_in,
                         n_out, info, plan, stream);
}

extern "C" int pesq_resample_plan_backward_pair(const float *grad_y0, float *grad_x0,
                                                const float *grad_y1, float *grad_x1,
                                                int64_t rows, int64_t n_in, int64_t n_out,
                                                const pesq_resample_plan_info *info,
                                                const void *plan, hipStream_t stream) {
    PESQ_CHECK_ARG(rows >= 0 && rows < (int64_t(1) << 40), "invalid row count %lld",
                   (long long)rows);
    return plan_backward(InRows{grad_y0, grad_y1, rows}, OutRows{grad_x0, grad_x1, rows},
                         2 * rows, n_in, n_out, info, plan, stream);
}
