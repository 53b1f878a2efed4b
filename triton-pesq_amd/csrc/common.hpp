// Shared device helpers of the PESQ HIP library (gfx950, wave64).
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>
#include <cstdio>

#include "pesq_hip.h"

namespace pesq {

constexpr int kWave = 64;

// Index of the calling wavefront in its workgroup, as a wave-uniform (scalar)
// value, so that frame and row indices derived from it stay in scalar
// registers and branches on them are uniform.
__device__ __forceinline__ int wave_index() {
    return __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x) / kWave);
}

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

// v of the lane `d` below in the same row of 16 lanes, 0 for the first d
// lanes of a row (DPP row shift, a VALU operation)
template <int d>
__device__ __forceinline__ double row_shr(double v) {
    static_assert(d >= 1 && d <= 15, "row shift");
    const int lo = __builtin_amdgcn_update_dpp(0, __double2loint(v), 0x110 + d, 0xF, 0xF, true);
    const int hi = __builtin_amdgcn_update_dpp(0, __double2hiint(v), 0x110 + d, 0xF, 0xF, true);
    return __hiloint2double(hi, lo);
}

// 64-bit DPP move with control kCtrl into the rows of kRowMask (0 elsewhere
// and where the source lane does not exist)
template <int kCtrl, int kRowMask>
__device__ __forceinline__ double dpp_move64(double v) {
    const int lo = __builtin_amdgcn_update_dpp(0, __double2loint(v), kCtrl, kRowMask, 0xF, true);
    const int hi = __builtin_amdgcn_update_dpp(0, __double2hiint(v), kCtrl, kRowMask, 0xF, true);
    return __hiloint2double(hi, lo);
}

// Inclusive prefix sum over the 64 lanes: Kogge-Stone within each row of 16
// lanes (row shifts 1, 2, 4, 8), then the last lane of rows 0 and 2 is added
// to rows 1 and 3 (row_bcast:15) and lane 31 to rows 2 and 3 (row_bcast:31).
// A fixed association order: bitwise deterministic.  All lanes active.
__device__ __forceinline__ double wave_inclusive_scan(double v) {
    v += row_shr<1>(v);
    v += row_shr<2>(v);
    v += row_shr<4>(v);
    v += row_shr<8>(v);
    v += dpp_move64<0x142, 0xA>(v);
    v += dpp_move64<0x143, 0xC>(v);
    return v;
}

// Ordering of LDS accesses within one wavefront: the accesses of a wavefront
// complete in program order, so when its lanes only exchange data among
// themselves a compiler level barrier between the write and the read phases
// is all the ordering needed.
__device__ __forceinline__ void wave_lds_fence() {
    __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
    __builtin_amdgcn_wave_barrier();
}

// Sums over the 64 lanes of K values per lane, through wave-private LDS
// (`red`: K rows of kWave + 4 doubles, so that the 16 lanes of an LDS cycle
// read distinct banks): lane 4 j + q adds value j of lanes q, q + 4, ...,
// q + 60 in that order and a quad DPP sum gives (p0 + p1) + (p2 + p3).  Sum j
// is returned in lanes 4 j .. 4 j + 3 (0 in lanes 4 K and above).  About 20
// VALU operations for all K sums, against some 20 per sum for a DPP tree.
// All 64 lanes must be active; `red` is free again when this returns.
template <int K>
__device__ __forceinline__ double wave_sums_lds(const double (&v)[K], double *red, int lane) {
    constexpr int kRow = kWave + 4;
    static_assert(4 * K <= kWave, "four lanes per sum");
#pragma unroll
    for (int j = 0; j < K; ++j) red[j * kRow + lane] = v[j];
    wave_lds_fence();
    const int j = lane / 4, q = lane % 4;
    double part = 0.0;
    if (j < K) {
        const double *src = red + j * kRow + q;
        part = src[0];
#pragma unroll
        for (int i = 1; i < kWave / 4; ++i) part += src[4 * i];
    }
    wave_lds_fence();
    part += dpp_move64<0xB1, 0xF>(part);  // quad_perm [1, 0, 3, 2]: + lane ^ 1
    part += dpp_move64<0x4E, 0xF>(part);  // quad_perm [2, 3, 0, 1]: + lane ^ 2
    return part;
}

// LDS doubles wave_sums_lds<K> needs per wavefront
template <int K>
constexpr int wave_sums_lds_doubles() {
    return K * (kWave + 4);
}

// v of the previous lane (0 in lane 0): DPP wave_shr:1
__device__ __forceinline__ double wave_shift_up(double v) { return dpp_move64<0x138, 0xF>(v); }

__device__ __forceinline__ double read_lane(double v, int lane) {
    return __hiloint2double(__builtin_amdgcn_readlane(__double2hiint(v), lane),
                            __builtin_amdgcn_readlane(__double2loint(v), lane));
}

// Sum over the 64 lanes, returned to every lane: an in-row scan by DPP row
// shifts leaves each row's sum in its last lane, and the four row sums are
// added in row order.  The association order is fixed, so the result is
// bitwise deterministic.  All 64 lanes must be active at the call.
__device__ __forceinline__ double wave_sum(double v) {
    v += row_shr<1>(v);
    v += row_shr<2>(v);
    v += row_shr<4>(v);
    v += row_shr<8>(v);
    return ((read_lane(v, 15) + read_lane(v, 31)) + read_lane(v, 47)) + read_lane(v, 63);
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

// x[n] for n < len, else 0, without a branch around the load (len >= 1): the
// index is clamped and the value selected, so that consecutive calls issue
// their loads back to back instead of waiting on each one.
__device__ __forceinline__ float load_or_zero(const float *x, int64_t n, int64_t len) {
    const float v = x[n < len ? n : len - 1];
    return n < len ? v : 0.0f;
}

// sum_{i < n} p[i * stride] accumulated in the order i = 0, 1, ..., n - 1
// (the same value as the plain loop), n >= 1.  The loads are issued in
// batches of 8 (indices past the end are clamped and their values dropped)
// so that a batch costs one memory latency instead of eight.
__device__ __forceinline__ double strided_sum(const double *p, int n, int64_t stride) {
    double s = 0.0;
    for (int i0 = 0; i0 < n; i0 += 8) {
        double v[8];
#pragma unroll
        for (int u = 0; u < 8; ++u) v[u] = p[int64_t(i0 + u < n ? i0 + u : n - 1) * stride];
#pragma unroll
        for (int u = 0; u < 8; ++u) {
            if (i0 + u < n) s += v[u];
        }
    }
    return s;
}

__host__ __device__ __forceinline__ int64_t cdiv(int64_t a, int64_t b) {
    return (a + b - 1) / b;
}

// Edge ramp of the pre-emphasis stage: samples 0..14 are weighted (k+1)/16,
// the last 15 samples (n-k)/16, both weights for rows shorter than 30, in the
// order head then tail.  Every factor is a small integer times 2^-4, so the
// products are exact; samples at least kEdge from both ends have weight 1.
constexpr int kEdge = 15;

__device__ __forceinline__ double edge_weight(int64_t n, int64_t len) {
    const int64_t head = n + 1 < 16 ? n + 1 : 16;
    const int64_t tail = len - n < 16 ? len - n : 16;
    return static_cast<double>(static_cast<int>(head)) * 0.0625 *
           (static_cast<double>(static_cast<int>(tail)) * 0.0625);
}

}  // namespace pesq
