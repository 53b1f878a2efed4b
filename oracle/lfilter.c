/*
 * Sequential IIR filter loops of the CPU oracle.  TEST INFRASTRUCTURE ONLY:
 * nothing in the shipped package links or loads this file.
 *
 * lfilter_df1_f32: torchaudio's float32 lfilter semantics as called by the
 *   reference (`torch_pesq/loss.py:159-161,199`; torchaudio
 *   `functional/filtering.py` `_lfilter`): the FIR part
 *   w[n] = sum_k b[k] x[n-k] / a[0] is formed first, then the all-pole part
 *   y[n] = w[n] - a[P] y[n-P] - ... - a[1] y[n-1] runs in float32, oldest tap
 *   first (the order of torchaudio's `lfilter_core` loop).  It is the CPU
 *   baseline's filter, not a parity oracle.
 *
 * lfilter_df2t_f64: the difference equation in float64, direct form II
 *   transposed with zero initial state (the form `scipy.signal.lfilter` uses).
 *
 * Both take `reverse`: filter the time reversed signal and write the result
 *   back reversed, which is the adjoint (vector-Jacobian product) of the
 *   causal filter.
 */

#include <stdint.h>
#include <stdlib.h>
#include <string.h>

static inline int64_t at(int64_t n, int64_t len, int reverse) {
    return reverse ? len - 1 - n : n;
}

void lfilter_df1_f32(const float *x, float *y, int64_t rows, int64_t len,
                     const float *b, const float *a, int64_t ncoef, int reverse) {
    float *w = (float *)malloc(sizeof(float) * (size_t)(len > 0 ? len : 1));
    const float a0 = a[0];
    for (int64_t r = 0; r < rows; ++r) {
        const float *xr = x + r * len;
        float *yr = y + r * len;
        for (int64_t n = 0; n < len; ++n) {
            float acc = 0.0f;
            for (int64_t k = ncoef - 1; k >= 0; --k) {
                if (n - k >= 0) acc += b[k] * xr[at(n - k, len, reverse)];
            }
            w[n] = acc / a0;
        }
        for (int64_t n = 0; n < len; ++n) {
            float acc = w[n];
            for (int64_t k = ncoef - 1; k >= 1; --k) {
                if (n - k >= 0) acc -= (a[k] / a0) * yr[at(n - k, len, reverse)];
            }
            yr[at(n, len, reverse)] = acc;
        }
    }
    free(w);
}

void lfilter_df2t_f64(const double *x, double *y, int64_t rows, int64_t len,
                      const double *b, const double *a, int64_t ncoef, int reverse) {
    double *state = (double *)calloc((size_t)(ncoef > 1 ? ncoef : 2), sizeof(double));
    const double a0 = a[0];
    for (int64_t r = 0; r < rows; ++r) {
        const double *xr = x + r * len;
        double *yr = y + r * len;
        memset(state, 0, sizeof(double) * (size_t)(ncoef > 1 ? ncoef : 2));
        for (int64_t n = 0; n < len; ++n) {
            const double xn = xr[at(n, len, reverse)];
            const double yn = (b[0] / a0) * xn + state[0];
            for (int64_t k = 1; k < ncoef; ++k) {
                const double next = (k + 1 < ncoef) ? state[k] : 0.0;
                state[k - 1] = next + (b[k] / a0) * xn - (a[k] / a0) * yn;
            }
            yr[at(n, len, reverse)] = yn;
        }
    }
    free(state);
}
