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

__global__ void __launch_bounds__(kResampleThreads)
    resample_fwd_kernel(const float *__restrict__ x, float *__restrict__ y, int64_t n_in,
                        int64_t n_out, const float *__restrict__ kernel,
                        const int32_t *__restrict__ tap_lo, const int32_t *__restrict__ tap_hi,
                        int64_t orig, int64_t nstep, int64_t width, int64_t wtotal,
                        int64_t blocks_per_row) {
    const int64_t row = blockIdx.x / blocks_per_row;
    const int64_t m = (blockIdx.x - row * blocks_per_row) * int64_t(blockDim.x) + threadIdx.x;
    if (m >= n_out) return;
    const int64_t l = m / nstep;
    const int64_t j = m - l * nstep;
    const float *xr = x + row * n_in;
    const float *kr = kernel + j * wtotal;
    const int64_t base = l * orig - width;
    const int lo = tap_lo[j], hi = tap_hi[j];
    double acc = 0.0;
    for (int k = lo; k < hi; ++k) {
        const int64_t i = base + k;
        if (i >= 0 && i < n_in) acc = fma(static_cast<double>(kr[k]), static_cast<double>(xr[i]), acc);
    }
    y[row * n_out + m] = static_cast<float>(acc);
}

__global__ void __launch_bounds__(kResampleThreads)
    resample_bwd_kernel(const float *__restrict__ gy, float *__restrict__ gx, int64_t n_in,
                        int64_t n_out, const float *__restrict__ kernel,
                        const int32_t *__restrict__ phase_lo, const int32_t *__restrict__ phase_hi,
                        int64_t orig, int64_t nstep, int64_t width, int64_t wtotal,
                        int64_t blocks_per_row) {
    const int64_t row = blockIdx.x / blocks_per_row;
    const int64_t i = (blockIdx.x - row * blocks_per_row) * int64_t(blockDim.x) + threadIdx.x;
    if (i >= n_in) return;
    const float *gr = gy + row * n_out;
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
    gx[row * n_in + i] = static_cast<float>(acc);
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

constexpr int kTileQ = 4;
constexpr int kTileOut = kResampleThreads * kTileQ;
constexpr int kMaxSpan = 8192;   // staged samples per workgroup (32 KiB)
constexpr int kMaxTable = 8192;  // tap table floats staged in LDS (32 KiB)

// where the forward reads its taps
enum TapSource { kTapsGlobal = 0, kTapsLds = 1, kTapsUniform = 2 };

template <int kSource>
__global__ void __launch_bounds__(kResampleThreads)
    resample_fwd_tiled(const float *__restrict__ x, float *__restrict__ y, int64_t n_in,
                       int64_t n_out, const float *__restrict__ taps,
                       const double *__restrict__ taps64, const int32_t *__restrict__ offs,
                       int orig, int nstep, int ntaps, int off_min, int span,
                       int64_t blocks_per_row) {
    extern __shared__ float lds[];
    float *xs = lds;
    float *tl = lds + span;
    const int64_t row = blockIdx.x / blocks_per_row;
    const int64_t m0 = (blockIdx.x - row * blocks_per_row) * kTileOut;
    const int64_t l_first = m0 / nstep;
    const int64_t in_lo = l_first * orig + off_min;
    const float *xr = x + row * n_in;
    for (int s = threadIdx.x; s < span; s += kResampleThreads) {
        const int64_t i = in_lo + s;
        xs[s] = (i >= 0 && i < n_in) ? xr[i] : 0.0f;
    }
    if constexpr (kSource == kTapsLds) {
        for (int s = threadIdx.x; s < ntaps * nstep; s += kResampleThreads) tl[s] = taps[s];
    }
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
    float *yr = y + row * n_out;
#pragma unroll
    for (int q = 0; q < kTileQ; ++q) {
        const int64_t m = m0 + threadIdx.x + int64_t(kResampleThreads) * q;
        if (m < n_out) yr[m] = static_cast<float>(acc[q]);
    }
}

// Adjoint of a single phase rate pair (new_step 1, integer decimation):
// thread u of the workgroup takes the orig consecutive inputs
// i = i0 + orig (u + 256 q) + c; input c of every thread uses the taps
// row[rho_c + s orig], rho_c = (c + width) mod orig, the same in every lane,
// read as float64 scalars.  The outputs go through LDS to be written with
// unit stride.
constexpr int kUniQ = 2;

__global__ void __launch_bounds__(kResampleThreads)
    resample_bwd_uniform(const float *__restrict__ gy, float *__restrict__ gx, int64_t n_in,
                         int64_t n_out, const double *__restrict__ row, int orig, int width,
                         int sweeps, int span, int64_t blocks_per_row) {
    extern __shared__ float lds[];
    float *gs = lds;
    float *out = lds + span;
    const int per_block = kResampleThreads * kUniQ * orig;
    const int64_t row_id = blockIdx.x / blocks_per_row;
    const int64_t i0 = (blockIdx.x - row_id * blocks_per_row) * per_block;
    const int64_t l_lo = (i0 + width) / orig - (sweeps - 1);
    const float *gr = gy + row_id * n_out;
    for (int s = threadIdx.x; s < span; s += kResampleThreads) {
        const int64_t m = l_lo + s;
        gs[s] = (m >= 0 && m < n_out) ? gr[m] : 0.0f;
    }
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
    float *gxr = gx + row_id * n_in;
    for (int s = threadIdx.x; s < per_block; s += kResampleThreads) {
        if (i0 + s < n_in) gxr[i0 + s] = out[s];
    }
}

template <bool kLds>
__global__ void __launch_bounds__(kResampleThreads)
    resample_bwd_tiled(const float *__restrict__ gy, float *__restrict__ gx, int64_t n_in,
                       int64_t n_out, const float *__restrict__ cols,
                       const int32_t *__restrict__ col_lo, int orig, int nstep, int width,
                       int nphases, int sweeps, int ncols, int span, int64_t blocks_per_row) {
    extern __shared__ float lds[];
    float *gs = lds;
    float *cl = lds + span;
    int32_t *clo = reinterpret_cast<int32_t *>(cl + nphases * ncols);
    const int64_t row = blockIdx.x / blocks_per_row;
    const int64_t i0 = (blockIdx.x - row * blocks_per_row) * kTileOut;
    const int64_t l_lo = (i0 + width) / orig - (sweeps - 1);
    const int64_t m_lo = l_lo * nstep;  // may be negative: those outputs read as zero
    const float *gr = gy + row * n_out;
    for (int s = threadIdx.x; s < span; s += kResampleThreads) {
        const int64_t m = m_lo + s;
        gs[s] = (m >= 0 && m < n_out) ? gr[m] : 0.0f;
    }
    if constexpr (kLds) {
        for (int s = threadIdx.x; s < nphases * ncols; s += kResampleThreads) cl[s] = cols[s];
        for (int s = threadIdx.x; s < ncols; s += kResampleThreads) clo[s] = col_lo[s];
    }
    __syncthreads();
    const float *cc = kLds ? cl : cols;
    const int32_t *cq = kLds ? clo : col_lo;
    float *gxr = gx + row * n_in;
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
                       dim3(kResampleThreads), 0, stream, x, y, n_in, n_out, kernel, tap_lo,
                       tap_hi, orig_step, new_step, width, width_total, bpr);
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
                       dim3(kResampleThreads), 0, stream, grad_y, grad_x, n_in, n_out, kernel,
                       phase_lo, phase_hi, orig_step, new_step, width, width_total, bpr);
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
    r.off_offs = align256(int64_t(taps) * nstep * sizeof(float));
    r.off_cols = r.off_offs + align256(int64_t(nstep) * sizeof(int32_t));
    r.off_col_lo = r.off_cols + align256(int64_t(phases) * ncols * sizeof(float));
    r.off_taps64 = r.off_col_lo + align256(int64_t(ncols) * sizeof(int32_t));
    r.off_row64 = r.off_taps64 + align256(int64_t(taps) * sizeof(double));
    r.bytes = r.off_row64 + align256(int64_t(ncols) * sizeof(double));
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
    return PESQ_OK;
}

extern "C" int pesq_resample_plan_forward(const float *x, float *y, int64_t rows, int64_t n_in,
                                          int64_t n_out, const pesq_resample_plan_info *info,
                                          const void *plan, hipStream_t stream) {
    PESQ_CHECK_ARG(info != nullptr, "null plan info");
    const pesq_resample_plan_info &r = *info;
    if (int st = check_resample(rows, n_in, n_out, r.orig_step, r.new_step, r.width, r.width_total)) {
        return st;
    }
    PESQ_CHECK_ARG(r.fwd_span > 0, "this rate pair has no tiled forward (window too wide)");
    if (rows == 0 || n_out == 0) return PESQ_OK;
    PESQ_CHECK_ARG(x && y && plan, "null pointer argument");
    // the base index of an output inside the staged window fits int32
    PESQ_CHECK_ARG(n_in < (int64_t(1) << 31) && n_out < (int64_t(1) << 31), "signal too long");
    const int64_t bpr = cdiv(n_out, kTileOut);
    PESQ_CHECK_ARG(rows * bpr < (int64_t(1) << 31), "too many rows x blocks for one launch");
    const unsigned char *base = static_cast<const unsigned char *>(plan);
    const float *taps = reinterpret_cast<const float *>(base);
    const double *taps64 = reinterpret_cast<const double *>(base + r.off_taps64);
    const int32_t *offs = reinterpret_cast<const int32_t *>(base + r.off_offs);
    const dim3 grid(static_cast<unsigned>(rows * bpr)), block(kResampleThreads);
    const size_t span_bytes = size_t(r.fwd_span) * sizeof(float);
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

extern "C" int pesq_resample_plan_backward(const float *grad_y, float *grad_x, int64_t rows,
                                           int64_t n_in, int64_t n_out,
                                           const pesq_resample_plan_info *info, const void *plan,
                                           hipStream_t stream) {
    PESQ_CHECK_ARG(info != nullptr, "null plan info");
    const pesq_resample_plan_info &r = *info;
    if (int st = check_resample(rows, n_in, n_out, r.orig_step, r.new_step, r.width, r.width_total)) {
        return st;
    }
    PESQ_CHECK_ARG(r.bwd_span > 0, "this rate pair has no tiled adjoint (window too wide)");
    if (rows == 0 || n_in == 0) return PESQ_OK;
    PESQ_CHECK_ARG(grad_y && grad_x && plan, "null pointer argument");
    PESQ_CHECK_ARG(n_in < (int64_t(1) << 31) && n_out < (int64_t(1) << 31), "signal too long");
    const int64_t bpr = cdiv(n_in, kTileOut);
    PESQ_CHECK_ARG(rows * bpr < (int64_t(1) << 31), "too many rows x blocks for one launch");
    const unsigned char *base = static_cast<const unsigned char *>(plan);
    if (r.new_step == 1) {
        const int64_t per_block = int64_t(kResampleThreads) * kUniQ * r.orig_step;
        const int64_t nb = cdiv(n_in, per_block);
        PESQ_CHECK_ARG(rows * nb < (int64_t(1) << 31), "too many rows x blocks for one launch");
        const size_t lds = size_t(r.bwd_span + per_block) * sizeof(float);
        hipLaunchKernelGGL(resample_bwd_uniform, dim3(static_cast<unsigned>(rows * nb)),
                           dim3(kResampleThreads), lds, stream, grad_y, grad_x, n_in, n_out,
                           reinterpret_cast<const double *>(base + r.off_row64), r.orig_step,
                           r.width, r.sweeps, r.bwd_span, nb);
        PESQ_CHECK_LAUNCH("resample backward (uniform)");
        return PESQ_OK;
    }
    const float *cols = reinterpret_cast<const float *>(base + r.off_cols);
    const int32_t *col_lo = reinterpret_cast<const int32_t *>(base + r.off_col_lo);
    const dim3 grid(static_cast<unsigned>(rows * bpr)), block(kResampleThreads);
    const size_t span_bytes = size_t(r.bwd_span) * sizeof(float);
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
