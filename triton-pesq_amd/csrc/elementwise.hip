// Stand-alone element-wise stages of the pipeline (the reference's
// triton_ops/elementwise.py operators): peak normalisation, edge ramp, level
// alignment scaling and the MOS epilogue, forward and backward.
//
// Reductions are two-stage with a fixed number of per row partials
// (kParts, one workgroup each, float64 accumulation) followed by a fixed
// order final sum in the consuming kernel: no atomics, bitwise reproducible.
#include <cmath>

#include "common.hpp"

namespace pesq {

constexpr int kParts = 64;       // partials per row
constexpr int kEwThreads = 256;  // threads per workgroup
constexpr int kEwSpan = 4096;    // samples per workgroup of the apply kernels

__device__ __forceinline__ double block_reduce_sum(double v, double *scratch) {
    v = wave_sum(v);
    const int wave = threadIdx.x / kWave;
    if (threadIdx.x % kWave == 0) scratch[wave] = v;
    __syncthreads();
    double total = 0.0;
    for (int i = 0; i < int(blockDim.x / kWave); ++i) total += scratch[i];
    return total;
}

__device__ __forceinline__ float block_reduce_max(float v, float *scratch) {
    v = wave_max(v);
    const int wave = threadIdx.x / kWave;
    if (threadIdx.x % kWave == 0) scratch[wave] = v;
    __syncthreads();
    float m = scratch[0];
    for (int i = 1; i < int(blockDim.x / kWave); ++i) m = fmaxf(m, scratch[i]);
    return m;
}

// -- peak normalisation ----------------------------------------------------

__global__ void __launch_bounds__(kEwThreads)
    peak_partial_kernel(const float *__restrict__ ref, const float *__restrict__ deg,
                        float *__restrict__ part, int64_t n) {
    __shared__ float scratch[kEwThreads / kWave];
    const int64_t b = blockIdx.x / kParts;
    const int c = blockIdx.x % kParts;
    const float *r = ref + b * n, *d = deg + b * n;
    float m = 0.0f;
    for (int64_t i = int64_t(c) * kEwThreads + threadIdx.x; i < n; i += int64_t(kParts) * kEwThreads) {
        m = fmaxf(m, fmaxf(fabsf(r[i]), fabsf(d[i])));
    }
    m = block_reduce_max(m, scratch);
    if (threadIdx.x == 0) part[b * kParts + c] = m;
}

__global__ void __launch_bounds__(kEwThreads)
    peak_apply_kernel(const float *__restrict__ part, const float *__restrict__ ref,
                      const float *__restrict__ deg, float *__restrict__ oref,
                      float *__restrict__ odeg, float *__restrict__ peak, int64_t n,
                      int64_t blocks_per_row) {
    const int64_t b = blockIdx.x / blocks_per_row;
    const int64_t blk = blockIdx.x - b * blocks_per_row;
    float m = part[b * kParts];
    for (int c = 1; c < kParts; ++c) m = fmaxf(m, part[b * kParts + c]);
    if (blk == 0 && threadIdx.x == 0) peak[b] = m;
    for (int64_t i = blk * kEwSpan + threadIdx.x; i < (blk + 1) * kEwSpan && i < n; i += kEwThreads) {
        oref[b * n + i] = __fdiv_rn(ref[b * n + i], m);
        odeg[b * n + i] = __fdiv_rn(deg[b * n + i], m);
    }
}

__global__ void __launch_bounds__(kEwThreads)
    div_rows_kernel(const float *__restrict__ g, const float *__restrict__ s, float *__restrict__ out,
                    int64_t n, int64_t blocks_per_row) {
    const int64_t b = blockIdx.x / blocks_per_row;
    const int64_t blk = blockIdx.x - b * blocks_per_row;
    const float m = s[b];
    for (int64_t i = blk * kEwSpan + threadIdx.x; i < (blk + 1) * kEwSpan && i < n; i += kEwThreads) {
        out[b * n + i] = __fdiv_rn(g[b * n + i], m);
    }
}

// -- edge ramp --------------------------------------------------------------

__global__ void __launch_bounds__(kEwThreads)
    edge_ramp_kernel(const float *__restrict__ x, float *__restrict__ y, int64_t n,
                     int64_t blocks_per_row) {
    const int64_t b = blockIdx.x / blocks_per_row;
    const int64_t blk = blockIdx.x - b * blocks_per_row;
    for (int64_t i = blk * kEwSpan + threadIdx.x; i < (blk + 1) * kEwSpan && i < n; i += kEwThreads) {
        // (x * head) * tail in float32; k/16 and j k/256 are exact
        const float head = i < 15 ? static_cast<float>(i + 1) / 16.0f : 1.0f;
        const float tail = i >= n - 15 ? static_cast<float>(n - i) / 16.0f : 1.0f;
        y[b * n + i] = (x[b * n + i] * head) * tail;
    }
}

// -- level alignment scaling -------------------------------------------------

__global__ void __launch_bounds__(kEwThreads)
    dot_partial_kernel(const float *__restrict__ a, const float *__restrict__ b,
                       double *__restrict__ part, int64_t n) {
    __shared__ double scratch[kEwThreads / kWave];
    const int64_t r = blockIdx.x / kParts;
    const int c = blockIdx.x % kParts;
    const float *x = a + r * n, *y = b + r * n;
    double acc = 0.0;
    for (int64_t i = int64_t(c) * kEwThreads + threadIdx.x; i < n; i += int64_t(kParts) * kEwThreads) {
        acc = fma(static_cast<double>(x[i]), static_cast<double>(y[i]), acc);
    }
    acc = block_reduce_sum(acc, scratch);
    if (threadIdx.x == 0) part[r * kParts + c] = acc;
}

__device__ __forceinline__ double sum_parts(const double *part, int64_t r) {
    double s = 0.0;
    for (int c = 0; c < kParts; ++c) s += part[r * kParts + c];
    return s;
}

// state[r] = {power, scale}; out = signal * scale
__global__ void __launch_bounds__(kEwThreads)
    align_apply_kernel(const double *__restrict__ part, const float *__restrict__ signal,
                       float *__restrict__ out, double *__restrict__ state, int64_t n_sig,
                       double denom, int64_t blocks_per_row) {
    const int64_t r = blockIdx.x / blocks_per_row;
    const int64_t blk = blockIdx.x - r * blocks_per_row;
    const double power = sum_parts(part, r) / denom / 1.04684;
    const double scale = sqrt(1e7 / power);
    if (blk == 0 && threadIdx.x == 0) {
        state[2 * r] = power;
        state[2 * r + 1] = scale;
    }
    for (int64_t i = blk * kEwSpan + threadIdx.x; i < (blk + 1) * kEwSpan && i < n_sig; i += kEwThreads) {
        out[r * n_sig + i] = static_cast<float>(static_cast<double>(signal[r * n_sig + i]) * scale);
    }
}

__global__ void __launch_bounds__(kEwThreads)
    align_grad_signal_kernel(const float *__restrict__ g, const double *__restrict__ state,
                             float *__restrict__ out, int64_t n, int64_t blocks_per_row) {
    const int64_t r = blockIdx.x / blocks_per_row;
    const int64_t blk = blockIdx.x - r * blocks_per_row;
    const double scale = state[2 * r + 1];
    for (int64_t i = blk * kEwSpan + threadIdx.x; i < (blk + 1) * kEwSpan && i < n; i += kEwThreads) {
        out[r * n + i] = static_cast<float>(static_cast<double>(g[r * n + i]) * scale);
    }
}

// d out / d filtered = 2 filtered (-0.5 S scale / power) / D, S = sum g signal
__global__ void __launch_bounds__(kEwThreads)
    align_grad_filtered_kernel(const double *__restrict__ part, const double *__restrict__ state,
                               const float *__restrict__ filtered, float *__restrict__ out,
                               int64_t n_flt, double denom, int64_t blocks_per_row) {
    const int64_t r = blockIdx.x / blocks_per_row;
    const int64_t blk = blockIdx.x - r * blocks_per_row;
    const double dot = sum_parts(part, r);
    const double power = state[2 * r], scale = state[2 * r + 1];
    const double coef = 2.0 * (-0.5 * dot * scale / power) / 1.04684 / denom;
    for (int64_t i = blk * kEwSpan + threadIdx.x; i < (blk + 1) * kEwSpan && i < n_flt; i += kEwThreads) {
        out[r * n_flt + i] = static_cast<float>(coef * static_cast<double>(filtered[r * n_flt + i]));
    }
}

// -- MOS epilogue -------------------------------------------------------------

__global__ void __launch_bounds__(kEwThreads)
    epilogue_kernel(const float *__restrict__ ds, const float *__restrict__ da, float *__restrict__ mos,
                    float *__restrict__ loss, double factor, int64_t batch) {
    const int64_t i = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
    if (i >= batch) return;
    const double s = ds[i], a = da[i];
    const double inner = 4.5 - 0.1 * s - 0.0309 * a;
    mos[i] = static_cast<float>(0.999 + 4.0 / (1.0 + exp(-1.3669 * inner + 3.8224)));
    loss[i] = static_cast<float>(factor * (0.1 * s + 0.0309 * a));
}

__global__ void __launch_bounds__(kEwThreads)
    epilogue_bwd_kernel(const float *__restrict__ ds, const float *__restrict__ da,
                        const float *__restrict__ gmos, const float *__restrict__ gloss,
                        float *__restrict__ gds, float *__restrict__ gda, double factor, int64_t batch) {
    const int64_t i = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
    if (i >= batch) return;
    double g_s = 0.0, g_a = 0.0;
    if (gmos) {
        const double inner = 4.5 - 0.1 * ds[i] - 0.0309 * da[i];
        const double ex = exp(-1.3669 * inner + 3.8224);
        const double dmos = 4.0 * 1.3669 * ex / ((1.0 + ex) * (1.0 + ex));
        g_s += gmos[i] * dmos * -0.1;
        g_a += gmos[i] * dmos * -0.0309;
    }
    if (gloss) {
        g_s += gloss[i] * factor * 0.1;
        g_a += gloss[i] * factor * 0.0309;
    }
    gds[i] = static_cast<float>(g_s);
    gda[i] = static_cast<float>(g_a);
}

}  // namespace pesq

using namespace pesq;

static int check_rows(int64_t rows, int64_t n) {
    PESQ_CHECK_ARG(rows >= 0 && n >= 0, "invalid sizes");
    PESQ_CHECK_ARG(n < (int64_t(1) << 40), "row too long");
    PESQ_CHECK_ARG(rows * kParts < (int64_t(1) << 31) && rows * cdiv(n, kEwSpan) < (int64_t(1) << 31),
                   "too many rows for one launch");
    return PESQ_OK;
}

static unsigned apply_grid(int64_t rows, int64_t n, int64_t &bpr) {
    bpr = cdiv(n, kEwSpan);
    return static_cast<unsigned>(rows * bpr);
}

extern "C" int pesq_elementwise_workspace(int64_t rows, size_t *bytes) {
    PESQ_CHECK_ARG(rows >= 0 && bytes, "invalid arguments");
    *bytes = size_t(rows) * kParts * sizeof(double) + size_t(rows) * 2 * sizeof(double);
    return PESQ_OK;
}

extern "C" int pesq_peak_normalize_forward(const float *ref, const float *deg, int64_t batch,
                                           int64_t len, float *out_ref, float *out_deg,
                                           float *peak, void *workspace, hipStream_t stream) {
    if (int st = check_rows(batch, len)) return st;
    PESQ_CHECK_ARG(len > 0, "peak_normalize needs at least one sample.");
    if (batch == 0) return PESQ_OK;
    PESQ_CHECK_ARG(ref && deg && out_ref && out_deg && peak && workspace, "null pointer argument");
    float *part = static_cast<float *>(workspace);
    hipLaunchKernelGGL(peak_partial_kernel, dim3(static_cast<unsigned>(batch * kParts)),
                       dim3(kEwThreads), 0, stream, ref, deg, part, len);
    PESQ_CHECK_LAUNCH("peak partial");
    int64_t bpr;
    hipLaunchKernelGGL(peak_apply_kernel, dim3(apply_grid(batch, len, bpr)), dim3(kEwThreads), 0,
                       stream, part, ref, deg, out_ref, out_deg, peak, len, bpr);
    PESQ_CHECK_LAUNCH("peak apply");
    return PESQ_OK;
}

extern "C" int pesq_peak_normalize_backward(const float *g_ref, const float *g_deg,
                                            const float *peak, int64_t batch, int64_t len,
                                            float *out_ref, float *out_deg, hipStream_t stream) {
    if (int st = check_rows(batch, len)) return st;
    if (batch == 0 || len == 0) return PESQ_OK;
    PESQ_CHECK_ARG(peak, "null peak");
    int64_t bpr;
    const unsigned grid = apply_grid(batch, len, bpr);
    if (g_ref && out_ref) {
        hipLaunchKernelGGL(div_rows_kernel, dim3(grid), dim3(kEwThreads), 0, stream, g_ref, peak,
                           out_ref, len, bpr);
        PESQ_CHECK_LAUNCH("peak backward (ref)");
    }
    if (g_deg && out_deg) {
        hipLaunchKernelGGL(div_rows_kernel, dim3(grid), dim3(kEwThreads), 0, stream, g_deg, peak,
                           out_deg, len, bpr);
        PESQ_CHECK_LAUNCH("peak backward (deg)");
    }
    return PESQ_OK;
}

extern "C" int pesq_edge_ramp(const float *x, float *y, int64_t rows, int64_t len,
                              hipStream_t stream) {
    if (int st = check_rows(rows, len)) return st;
    PESQ_CHECK_ARG(len >= 15,
                   "edge_ramp needs at least 15 samples, the length of a single ramp, got %lld",
                   (long long)len);
    if (rows == 0) return PESQ_OK;
    PESQ_CHECK_ARG(x && y, "null pointer argument");
    int64_t bpr;
    hipLaunchKernelGGL(edge_ramp_kernel, dim3(apply_grid(rows, len, bpr)), dim3(kEwThreads), 0,
                       stream, x, y, len, bpr);
    PESQ_CHECK_LAUNCH("edge ramp");
    return PESQ_OK;
}

extern "C" int pesq_align_scale_forward(const float *signal, const float *filtered, int64_t rows,
                                        int64_t n_sig, int64_t n_flt, float *out, double *state,
                                        void *workspace, hipStream_t stream) {
    if (int st = check_rows(rows, n_sig > n_flt ? n_sig : n_flt)) return st;
    PESQ_CHECK_ARG(n_sig > 0 && n_flt > 0, "align_scale needs at least one sample.");
    if (rows == 0) return PESQ_OK;
    PESQ_CHECK_ARG(signal && filtered && out && state && workspace, "null pointer argument");
    double *part = static_cast<double *>(workspace);
    hipLaunchKernelGGL(dot_partial_kernel, dim3(static_cast<unsigned>(rows * kParts)),
                       dim3(kEwThreads), 0, stream, filtered, filtered, part, n_flt);
    PESQ_CHECK_LAUNCH("align power");
    int64_t bpr;
    hipLaunchKernelGGL(align_apply_kernel, dim3(apply_grid(rows, n_sig, bpr)), dim3(kEwThreads), 0,
                       stream, part, signal, out, state, n_sig, static_cast<double>(n_flt + 5120),
                       bpr);
    PESQ_CHECK_LAUNCH("align apply");
    return PESQ_OK;
}

extern "C" int pesq_align_scale_backward(const float *grad, const float *signal,
                                         const float *filtered, const double *state, int64_t rows,
                                         int64_t n_sig, int64_t n_flt, float *g_signal,
                                         float *g_filtered, void *workspace, hipStream_t stream) {
    if (int st = check_rows(rows, n_sig > n_flt ? n_sig : n_flt)) return st;
    if (rows == 0) return PESQ_OK;
    PESQ_CHECK_ARG(grad && state, "null pointer argument");
    int64_t bpr;
    if (g_signal) {
        hipLaunchKernelGGL(align_grad_signal_kernel, dim3(apply_grid(rows, n_sig, bpr)),
                           dim3(kEwThreads), 0, stream, grad, state, g_signal, n_sig, bpr);
        PESQ_CHECK_LAUNCH("align backward (signal)");
    }
    if (g_filtered) {
        PESQ_CHECK_ARG(signal && filtered && workspace, "null pointer argument");
        double *part = static_cast<double *>(workspace);
        hipLaunchKernelGGL(dot_partial_kernel, dim3(static_cast<unsigned>(rows * kParts)),
                           dim3(kEwThreads), 0, stream, grad, signal, part, n_sig);
        PESQ_CHECK_LAUNCH("align backward dot");
        hipLaunchKernelGGL(align_grad_filtered_kernel, dim3(apply_grid(rows, n_flt, bpr)),
                           dim3(kEwThreads), 0, stream, part, state, filtered, g_filtered, n_flt,
                           static_cast<double>(n_flt + 5120), bpr);
        PESQ_CHECK_LAUNCH("align backward (filtered)");
    }
    return PESQ_OK;
}

extern "C" int pesq_epilogue_forward(const float *d_symm, const float *d_asymm, int64_t batch,
                                     double factor, float *mos, float *loss, hipStream_t stream) {
    PESQ_CHECK_ARG(batch >= 0, "invalid batch");
    if (batch == 0) return PESQ_OK;
    PESQ_CHECK_ARG(d_symm && d_asymm && mos && loss, "null pointer argument");
    hipLaunchKernelGGL(epilogue_kernel, dim3(static_cast<unsigned>(cdiv(batch, kEwThreads))),
                       dim3(kEwThreads), 0, stream, d_symm, d_asymm, mos, loss, factor, batch);
    PESQ_CHECK_LAUNCH("epilogue");
    return PESQ_OK;
}

extern "C" int pesq_epilogue_backward(const float *d_symm, const float *d_asymm, const float *g_mos,
                                      const float *g_loss, int64_t batch, double factor,
                                      float *g_symm, float *g_asymm, hipStream_t stream) {
    PESQ_CHECK_ARG(batch >= 0, "invalid batch");
    if (batch == 0) return PESQ_OK;
    PESQ_CHECK_ARG(d_symm && d_asymm && g_symm && g_asymm, "null pointer argument");
    hipLaunchKernelGGL(epilogue_bwd_kernel, dim3(static_cast<unsigned>(cdiv(batch, kEwThreads))),
                       dim3(kEwThreads), 0, stream, d_symm, d_asymm, g_mos, g_loss, g_symm,
                       g_asymm, factor, batch);
    PESQ_CHECK_LAUNCH("epilogue backward");
    return PESQ_OK;
}
