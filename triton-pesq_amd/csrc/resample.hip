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
