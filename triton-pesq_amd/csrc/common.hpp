// Shared device helpers of the PESQ HIP library (gfx950, wave64).
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>
#include <cstdio>

#include "pesq_hip.h"

namespace pesq {

constexpr int kWave = 64;

// ---------------------------------------------------------------------------
// status / error string (host side)
// ---------------------------------------------------------------------------

void set_error(const char *fmt, ...);

#define PESQ_CHECK_ARG(cond, ...)                                              \
    do {                                                                       \
        if (!(cond)) {                                                         \
            ::pesq::set_error(__VA_ARGS__);                                    \
            return PESQ_ERR_ARGUMENT;                                          \
        }                                                                      \
    } while (0)

#define PESQ_CHECK_LAUNCH(what)                                                \
    do {                                                                       \
        hipError_t err_ = hipGetLastError();                                   \
        if (err_ != hipSuccess) {                                              \
            ::pesq::set_error("%s: %s", what, hipGetErrorString(err_));        \
            return PESQ_ERR_HIP;                                               \
        }                                                                      \
    } while (0)

// ---------------------------------------------------------------------------
// wave-level primitives
// ---------------------------------------------------------------------------

__device__ __forceinline__ int lane_id() { return __lane_id(); }

__device__ __forceinline__ double shfl_up(double v, int d) {
    return __shfl_up(v, static_cast<unsigned>(d), kWave);
}

__device__ __forceinline__ double shfl_xor(double v, int m) {
    return __shfl_xor(v, m, kWave);
}

__device__ __forceinline__ float shfl_xor(float v, int m) {
    return __shfl_xor(v, m, kWave);
}

__device__ __forceinline__ double shfl(double v, int src) {
    return __shfl(v, src, kWave);
}

// Butterfly sum over the 64 lanes; every lane ends with the same value and
// the association order is fixed, so the result is bitwise deterministic.
__device__ __forceinline__ double wave_sum(double v) {
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) v += shfl_xor(v, m);
    return v;
}

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) v = fmaxf(v, shfl_xor(v, m));
    return v;
}

__device__ __forceinline__ double wave_max(double v) {
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) v = fmax(v, shfl_xor(v, m));
    return v;
}

__host__ __device__ __forceinline__ int64_t cdiv(int64_t a, int64_t b) {
    return (a + b - 1) / b;
}

// Edge ramp of the pre-emphasis stage: samples 0..14 are weighted (k+1)/16,
// the last 15 samples (n-k)/16, both weights for rows shorter than 30, in the
// order head then tail.
__device__ __forceinline__ double edge_weight(int64_t n, int64_t len) {
    double w = 1.0;
    if (n < 15) w = static_cast<double>(n + 1) * 0.0625;
    if (n >= len - 15) w *= static_cast<double>(len - n) * 0.0625;
    return w;
}

}  // namespace pesq
