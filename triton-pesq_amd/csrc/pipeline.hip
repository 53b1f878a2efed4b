// Fused PESQ pipeline, forward and backward, for 16 kHz rows.
//
// Forward (5 kernels):
//   1. iir_aggregate  <power, pre>   per block end states of both filters on the
//                                    raw inputs
//   2. iir_output     <power, pre>   p = pre(ramp(s)), f = power(s) (kept when a
//                                    gradient is needed), per block sum f^2
//   3. stft_fwd       per (item, 16 frames): frames of scale * p, FFT, |X|^2,
//                                    Bark sums, silent frames, band partials
//   4. chain_fwd      per (item, 16 frames): band and frame equalisation,
//                                    loudness, disturbance, per frame distances
//   5. chain_final    per item: overlapping sums, distances, MOS, loss
// Backward (4 kernels):
//   6. chain_bwd      per (item, 16 frames): adjoint of 4 and of the PSQM/MOS
//   7. stft_bwd       per (grad row, 7 hop blocks): band ratio adjoint, frame
//                                    spectra recomputed, adjoint FFT, overlap-add
//   8. iir_aggregate  <power^T, pre^T> on (f, dL/dp), time reversed
//   9. iir_output     <power^T, pre^T> and the level alignment adjoint:
//        dL/ds = scale ramp(pre^T g_p) - scale S / E power^T f,  S = sum g_p p
// Each scan pass also runs iir_prefix (block start states from the block
// aggregates) between its aggregate and output kernels.
//
// The level alignment (torch_pesq/loss.py:127-139) is folded in: with
// E = sum f^2 the aligned, pre-emphasised signal is p_aligned = scale * p,
// scale = sqrt(1e7 (len + 5120) 1.04684 / E), because the ramp and the
// pre-emphasis filter are linear.  The peak normalisation that precedes it
// (torch_pesq/loss.py:179-183) multiplies s by 1 / peak, which scales p by
// 1 / peak and scale by peak: p_aligned does not depend on it, so the scans
// run on the raw signal s and the peak is never formed.  (Its gradient path
// is zero for the same reason: the loss is invariant under s -> c s.)
#include <cmath>

#include <algorithm>
#include <string>
#include <type_traits>

#include "pipeline_layout.hpp"
#include "tables.hpp"

namespace pesq {


// ---------------------------------------------------------------------------
// IIR modes
// ---------------------------------------------------------------------------

struct PipeFwdMode {
    static constexpr int kInputs = 1;
    static constexpr int kOutputs = 2;  // p, f
    static constexpr bool kRamp = true;
    static constexpr bool kReverse = false;
    static constexpr bool kAccumulates = true;
    static constexpr bool kB2 = false;
    using In = float;
    using Out = float;

    const float *ref, *deg;
    float *p, *f;             // outputs; f may be null
    double *energy;           // [rows, nblk]
    int64_t len;
    int batch, nblk, row0, nrg;

    __device__ __forceinline__ const float *src(int row, int) const {
        return row < batch ? ref + int64_t(row) * len : deg + int64_t(row - batch) * len;
    }
    __device__ __forceinline__ float *dst(int row, int q) const {
        if (q == 0) return p + int64_t(row) * len;
        return f != nullptr && row >= row0 && row < row0 + nrg ? f + int64_t(row - row0) * len
                                                               : nullptr;
    }
    // filter A (level alignment band pass) sees the signal, filter B
    // (pre-emphasis) the edge ramped signal
    __device__ __forceinline__ void inputs(double w, const float *in, double &xa,
                                           double &xb) const {
        xa = in[0];
        xb = static_cast<double>(in[0]) * w;
    }
    __device__ __forceinline__ void setup(int, double *, int) const {}
    __device__ __forceinline__ void compute(double, double ya, double yb, double &acc,
                                            const double *, float *out) const {
        out[0] = static_cast<float>(yb);
        out[1] = static_cast<float>(ya);
        acc = fma(ya, ya, acc);
    }
    __device__ __forceinline__ void finish(int row, int blk, double total) const {
        energy[int64_t(row) * nblk + blk] = total;
    }
};

struct PipeBwdMode {
    static constexpr int kInputs = 2;
    static constexpr int kOutputs = 1;
    static constexpr bool kRamp = true;
    static constexpr bool kReverse = true;
    static constexpr bool kAccumulates = false;
    static constexpr bool kB2 = false;
    using In = float;
    using Out = float;

    const float *f, *gp;      // [nrg, len] each
    const double *rowconst;   // [rows, 4]: -, E, scale, -
    const double *spart;      // [nrg, nhop]
    float *g_ref, *g_deg;
    int64_t len;
    int batch, row0, nhop;

    // filter A (power^T) runs on f, filter B (pre^T) on dL/dp
    __device__ __forceinline__ const float *src(int row, int q) const {
        return (q == 0 ? f : gp) + int64_t(row) * len;
    }
    __device__ __forceinline__ float *dst(int row, int) const {
        const int stacked = row0 + row;
        return stacked < batch ? g_ref + int64_t(stacked) * len
                               : g_deg + int64_t(stacked - batch) * len;
    }
    __device__ __forceinline__ void inputs(double, const float *in, double &xa, double &xb) const {
        xa = in[0];
        xb = in[1];
    }
    // scale and scale S / E, S = sum of the per hop block partials of dL/dp . p
    // (lane l sums partials l, l + 64, ...: the first 8 are requested by
    // prefetch, any further ones here, in the order of strided_sum)
    struct Pre {
        double v[8];
    };
    __device__ __forceinline__ int mine(int lane) const {
        return lane < nhop ? (nhop - 1 - lane) / kWave + 1 : 0;
    }
    __device__ __forceinline__ void prefetch(int row, int lane, Pre &pre) const {
        const int n = mine(lane);
        const double *src = spart + int64_t(row) * nhop + (lane < nhop ? lane : 0);
#pragma unroll
        for (int u = 0; u < 8; ++u) {
            pre.v[u] = src[int64_t(u < n ? u : (n > 0 ? n - 1 : 0)) * kWave];
        }
    }
    __device__ __forceinline__ void setup(int row, double *sh, int lane, const Pre &pre) const {
        const int n = mine(lane);
        double s = 0.0;
#pragma unroll
        for (int u = 0; u < 8; ++u) {
            if (u < n) s += pre.v[u];
        }
        if (n > 8) {
            const double *src = spart + int64_t(row) * nhop + lane;
            for (int i0 = 8; i0 < n; i0 += 8) {
                double v[8];
#pragma unroll
                for (int u = 0; u < 8; ++u) {
                    v[u] = src[int64_t(i0 + u < n ? i0 + u : n - 1) * kWave];
                }
#pragma unroll
                for (int u = 0; u < 8; ++u) {
                    if (i0 + u < n) s += v[u];
                }
            }
        }
        s = wave_sum(s);
        const double *rc = rowconst + int64_t(row0 + row) * 4;
        sh[1] = rc[2];
        sh[2] = rc[2] * s / rc[1];
    }
    __device__ __forceinline__ void compute(double w, double ya, double yb, double &,
                                            const double *sh, float *out) const {
        out[0] = static_cast<float>(sh[1] * w * yb - sh[2] * ya);
    }
    __device__ __forceinline__ void finish(int, int, double) const {}
};

// The level alignment filter (power^T on f) of the backward scan alone, for
// its aggregate pass inside the forward's STFT kernel (iir.hpp
// aggregate_block over sections 0 .. 4); same input and time order as
// PipeBwdMode, no outputs.
struct PipeBwdPowerMode {
    static constexpr int kInputs = 1;
    static constexpr int kOutputs = 1;
    static constexpr bool kRamp = false;
    static constexpr bool kReverse = true;
    static constexpr bool kAccumulates = false;
    static constexpr bool kB2 = false;
    using In = float;
    using Out = float;

    const float *f;  // [nrg, len]
    int64_t len;

    __device__ __forceinline__ const float *src(int row, int) const { return f + int64_t(row) * len; }
    __device__ __forceinline__ void inputs(double, const float *in, double &xa, double &xb) const {
        xa = in[0];
        xb = 0.0;
    }
};

// ---------------------------------------------------------------------------
// shared chain helpers
// ---------------------------------------------------------------------------

struct PipeArgs {
    const ModelTable *tab;
    const float *ref, *deg;
    unsigned char *ws;  // forward workspace
    unsigned char *bw;  // backward workspace
    PipeLayout L;
    double factor;
    float *d_symm, *d_asymm, *mos, *loss;  // mos / loss may be null
    const float *g_symm, *g_asymm, *g_mos, *g_loss;
    // Bark spectra read by the chain kernels and the gradients they write,
    // [batch, frames, 49] each (inside the workspaces for the pipeline)
    const float *bark_ref, *bark_deg;
    float *gbark_ref, *gbark_deg;
};

template <typename T>
__host__ __device__ __forceinline__ T *region(unsigned char *base, size_t off) {
    return reinterpret_cast<T *>(base + off);
}

__device__ __forceinline__ double *frame_array(const PipeArgs &a, int which) {
    return region<double>(a.ws, a.L.frame) + int64_t(which) * a.L.batch * a.L.frames;
}

// What the backward needs of a (frame, band) of the forward chain, stored in
// float32 (16 bytes instead of the three float64 values it derives them from):
//   dist   the clamped disturbance sign(u) max(|u| - 0.25 min(L_d, L_r), 0);
//          its sign is sign(u) wherever it is non-zero, and where it is zero
//          the band adds nothing to either norm's gradient, so the backward
//          takes every decision of the dead zone (sign, zone, which loudness
//          is the smaller) from it and none from rounded loudnesses
//   asc    the raw asymmetry factor where it lies in [3, 12] (the factor and
//          its log-derivative both count), -12 where it is capped, 0 where
//          it is cut: the clamp decisions are the forward's
//   sr, sd d L_r / d equ_ref and d L_d / d equ_deg at this (frame, band)
// Each is the float64 value rounded once, so a gradient term carries float32
// rounding of itself, not of a difference of loudnesses.
struct alignas(16) ChainTerms {
    float dist, asc, sr, sd;
};
static_assert(sizeof(ChainTerms) == kChainTermBytes, "float4 layout");

__device__ __forceinline__ ChainTerms *chain_terms(const PipeArgs &a) {
    return region<ChainTerms>(a.ws, a.L.loud);
}

__device__ __forceinline__ double *band_array(const PipeArgs &a, int which) {
    return region<double>(a.ws, a.L.band) + int64_t(which) * a.L.batch * a.L.nb;
}

// Band `band` of the per tile band partials base[tile][nb], summed over tiles
// part, part + parts, part + 2 parts, ... (in that order); 0 when there are none.
__device__ __forceinline__ double tile_partial(const double *base, int64_t ntile, int part,
                                               int parts, int band, int nb) {
    const int n = ntile > part ? static_cast<int>((ntile - 1 - part) / parts) + 1 : 0;
    return n > 0 ? strided_sum(base + int64_t(part) * nb + band, n, int64_t(parts) * nb) : 0.0;
}

// K sums s_k = sum_{i < n_k} p_k[i * stride], each accumulated in the order
// i = 0, 1, ... (the value of strided_sum), with the loads of all K sums
// issued together, kRound per sum at a time, so that they share one memory
// latency per round.  A sum with n_k = 0 is 0 and loads nothing.
template <int K, int kRound = 2>
__device__ __forceinline__ void strided_sums(const double *const (&p)[K], const int (&n)[K],
                                             int64_t stride, double (&out)[K]) {
    int nmax = 0;
#pragma unroll
    for (int k = 0; k < K; ++k) {
        out[k] = 0.0;
        nmax = n[k] > nmax ? n[k] : nmax;
    }
    for (int i0 = 0; i0 < nmax; i0 += kRound) {
        double v[K][kRound];
#pragma unroll
        for (int k = 0; k < K; ++k) {
#pragma unroll
            for (int u = 0; u < kRound; ++u) {
                const int i = i0 + u < n[k] ? i0 + u : n[k] - 1;  // clamped, value dropped
                v[k][u] = n[k] > 0 ? p[k][int64_t(i) * stride] : 0.0;
            }
        }
#pragma unroll
        for (int k = 0; k < K; ++k) {
#pragma unroll
            for (int u = 0; u < kRound; ++u) {
                if (i0 + u < n[k]) out[k] += v[k][u];
            }
        }
    }
}

// exp and expm1 for the chain, from the mathematics, for |x| < 700 (the
// chain's arguments stay far from overflow, underflow and special values):
// x = k ln2 + r with k = rint(x / ln2), |r| <= ln2 / 2, r formed in two steps
// with ln2 split into a 33-bit head (k ln2_hi is exact for |k| < 2^20) and a
// tail; e^r - 1 = r Q(r) with Q the Taylor series of (e^r - 1) / r to degree 12
// (the first dropped term, r^13 / 14!, is below 5e-18); then
// exp(x) = 2^k + 2^k r Q(r) and expm1(x) = (2^k - 1) + 2^k r Q(r), one fused
// multiply-add each (expm1 keeps full relative precision near 0, where k = 0).
// Within 3e-16 relative of the exact values, in about 20 operations against
// the library's 53.
struct ExpParts {
    double two_k;  // 2^k
    double p;      // e^r - 1
};

__device__ __forceinline__ ExpParts exp_parts(double x) {
    constexpr double kInvLn2 = 0x1.71547652b82fep+0;  // 1 / ln 2
    constexpr double kLn2Hi = 0x1.62e42fef00000p-1;   // ln 2, first 33 bits
    constexpr double kLn2Lo = 0x1.473de6af278edp-34;  // ln 2 - kLn2Hi
    const double kf = rint(x * kInvLn2);
    double r = fma(-kf, kLn2Hi, x);
    r = fma(-kf, kLn2Lo, r);
    double q = 1.0 / 6227020800.0;  // 1 / 13!
    q = fma(q, r, 1.0 / 479001600.0);
    q = fma(q, r, 1.0 / 39916800.0);
    q = fma(q, r, 1.0 / 3628800.0);
    q = fma(q, r, 1.0 / 362880.0);
    q = fma(q, r, 1.0 / 40320.0);
    q = fma(q, r, 1.0 / 5040.0);
    q = fma(q, r, 1.0 / 720.0);
    q = fma(q, r, 1.0 / 120.0);
    q = fma(q, r, 1.0 / 24.0);
    q = fma(q, r, 1.0 / 6.0);
    q = fma(q, r, 0.5);
    q = fma(q, r, 1.0);
    return {ldexp(1.0, static_cast<int>(kf)), r * q};
}

__device__ __forceinline__ double exp_chain(double x) {
    const ExpParts e = exp_parts(x);
    return fma(e.two_k, e.p, e.two_k);
}

__device__ __forceinline__ double expm1_chain(double x) {
    const ExpParts e = exp_parts(x);
    return fma(e.two_k, e.p, e.two_k - 1.0);
}

// Logarithms for the chain, to about 1e-13 relative: a float32 estimate y0
// (hardware log) refined by one float64 Newton step on the exponential,
// y1 = y0 - f(y0) / f'(y0), whose error is about half the square of the
// estimate's (1e-7 relative).  The step costs one exp or expm1 (about 20
// operations), against 135 for the library's float64 log; the
// estimate and the correction term need only float32 relative accuracy, so
// their divisions are hardware float32 reciprocals (1 ulp).

// log(1 + u) for u > 0 (u < 3e38).  The estimate is Kahan's
// log1p(u) = log(w) u / (w - 1), w = 1 + u in float32 (u itself when w
// rounds to 1), accurate to a few float32 units for every u; the step is
// y <- y - (expm1(y) - u) / (1 + expm1(y)).
__device__ __forceinline__ double log1p_refined(double u) {
    const float uf = static_cast<float>(u);
    const float w = 1.0f + uf;
    const float y0 = w == 1.0f ? uf : __logf(w) * (uf * __builtin_amdgcn_rcpf(w - 1.0f));
    const double y = static_cast<double>(y0);
    const double m = expm1_chain(y);
    return y - (m - u) * static_cast<double>(__builtin_amdgcn_rcpf(static_cast<float>(1.0 + m)));
}

// log(num / den) for num, den > 0 with a float32-range quotient; the step is
// y <- y + (num exp(-y) - den) / den.
__device__ __forceinline__ double log_ratio_refined(double num, double den) {
    const float inv_den = __builtin_amdgcn_rcpf(static_cast<float>(den));
    const double y = static_cast<double>(__logf(static_cast<float>(num) * inv_den));
    return y + (num * exp_chain(-y) - den) * static_cast<double>(inv_den);
}

// Zwicker loudness sl (2 th)^e ((0.5 + 0.5 x / th)^e - 1) above the threshold,
// written as loud_scale expm1(e log1p((x - th) / (2 th))) so that bands just
// above their threshold keep full precision (inv2th = 1 / (2 th)).
__device__ __forceinline__ double loudness(double x, double th, double inv2th, double e,
                                           double ls) {
    if (!(x > th)) return 0.0;
    return ls * expm1_chain(e * log1p_refined((x - th) * inv2th));
}

// d loudness / dx from the loudness l itself: with 1 + u = (x + th) / (2 th),
// l = ls ((1 + u)^e - 1) gives ls e (1 + u)^(e - 1) / (2 th) = e (l + ls) / (x + th);
// to float32 accuracy (the precision it is stored in): the quotient through
// the hardware reciprocal (1 ulp)
__device__ __forceinline__ float loudness_slope(double x, double l, double th, double e,
                                                double ls) {
    return x > th ? static_cast<float>(e * (l + ls)) *
                        __builtin_amdgcn_rcpf(static_cast<float>(x + th))
                  : 0.0f;
}

// raw asymmetry factor ((ed + 50) / (er + 50))^1.2 = z^6 with z the fifth
// root of the ratio num / den: a float32 estimate z0 = 2^(log2(q) / 5) of the
// float32 quotient q (hardware log2 and exp2, about 5e-7 relative), then one
// float64 Newton step on f(z) = den z^5 - num, z1 = z0 - f(z0) / f'(z0), whose
// error is about twice the square of the estimate's; the correction term
// needs only float32 relative accuracy, so f'(z0) is inverted in float32.
// About 1e-11 relative for z1^6, in 21 operations against about 50 for the
// logarithm and exponential.  num, den >= 50 (energies are non-negative) with
// a float32-range quotient.  The backward reads the forward's values, so the
// clamp decisions (below 3, above 12) agree.
__device__ __forceinline__ double asymmetry(double ed, double er) {
    const double num = ed + 50.0, den = er + 50.0;
    const float q = static_cast<float>(num) * __builtin_amdgcn_rcpf(static_cast<float>(den));
    const double z0 = static_cast<double>(__builtin_amdgcn_exp2f(0.2f * __builtin_amdgcn_logf(q)));
    const double z2 = z0 * z0;
    const double dz4 = den * (z2 * z2);
    const double f = fma(dz4, z0, -num);
    const double inv_fp = static_cast<double>(__builtin_amdgcn_rcpf(static_cast<float>(5.0 * dz4)));
    const double z = fma(-f, inv_fp, z0);
    const double s2 = z * z;
    return s2 * s2 * s2;
}

__device__ __forceinline__ double sgn(double v) { return v > 0.0 ? 1.0 : (v < 0.0 ? -1.0 : 0.0); }

// ---------------------------------------------------------------------------
// 3. STFT forward + silent frames + band partials, per (item, 16 frames)
// ---------------------------------------------------------------------------

constexpr int kStftWaves = 8;

// kLean: the variant for grids of several workgroups per CU, which keeps
// fewer values live (no next-frame prefetch, twiddles read again per frame,
// a rolled band sum) so that more wavefronts fit per SIMD.
template <typename real, bool kLean, int kWaves = kStftWaves>
__global__ void __launch_bounds__(kWave *kWaves, kLean ? 4 : 1) stft_fwd_kernel(PipeArgs a) {
#pragma clang fp contract(off)  // the same bits in both variants (spectral.hpp)
    constexpr int kSideWaves = kWaves / 2;            // wavefronts per side
    constexpr int kPerWave = 2 * kTile / kWaves;      // frames per wavefront
    static_assert(kSideWaves * kPerWave == kTile, "a tile per side");
    __shared__ cplx<real> fftbuf[kWaves][kHalf];
    __shared__ float barks[2][kTile][kBands];
    __shared__ float keepflag[kTile];
    // kLean: the twiddle tables (kHalf entries each) and the window, staged
    // once per workgroup and read per frame (10 KB; two workgroups per CU
    // still fit)
    using T2 = typename Vec2<real>::type;
    __shared__ T2 lds_pass[kLean ? kPassTwiddles : 1], lds_tw512[kLean ? kHalf : 1];
    __shared__ float lds_win[kLean ? kNfft : 1];

    const ModelTable &t = *a.tab;
    const PipeLayout &L = a.L;
    const int item = blockIdx.x / L.ntile;
    const int tile = blockIdx.x - item * L.ntile;
    const int t0 = tile * kTile;
    const int wave = wave_index();
    const int lane = threadIdx.x % kWave;
    if constexpr (!kLean) {
        if (L.host_power && blockIdx.x >= L.batch * L.ntile) {
            // workgroups past the transform's: the aggregate pass of the
            // backward's level alignment filter on f (which the scan has just
            // written), a block of a gradient row per wavefront
            const int64_t g = int64_t(blockIdx.x - L.batch * L.ntile) * kWaves + wave;
            if (g < L.nrg * L.nblk) {
                const int row = static_cast<int>(g / L.nblk);
                const int blk = static_cast<int>(g - int64_t(row) * L.nblk);
                double *aggr = region<double>(a.ws, L.aggr_b);
                double *lanes = aggr + scan_aggr_doubles(L.nrg, L.nblk, kPipeSections);
                const PipeBwdPowerMode m{region<float>(a.ws, L.f), L.len};
                aggregate_block<kPowerSections, 0, 0, kPipeSections>(
                    m, t.iir, aggr, lanes, L.len, static_cast<int>(L.nblk), row, blk, lane);
            }
            return;
        }
    }
    const int side = wave / kSideWaves;          // 0 = reference, 1 = degraded
    const int row = side * L.batch + item;

    // samples of this wavefront's first frame, requested before anything else
    const float *p = region<float>(a.ws, L.p) + int64_t(row) * L.len;
    const int64_t f_first = t0 + (wave % kSideWaves) * kPerWave;
    float cur[8];
    load_frame(p, (f_first < L.frames ? f_first : L.frames - 1) * kHop, L.len, lane, cur);

    // row constants: -, E, scale, -
    const double *energy = region<double>(a.ws, L.energy) + int64_t(row) * L.nblk;
    const int nmine = lane < L.nblk ? static_cast<int>((L.nblk - 1 - lane) / kWave + 1) : 0;
    double e = nmine > 0 ? strided_sum(energy + lane, nmine, kWave) : 0.0;
    e = wave_sum(e);
    const double power = e / static_cast<double>(L.len + 5120) / 1.04684;
    const double scale = sqrt(1e7 / power);
    if (tile == 0 && wave % kSideWaves == 0 && lane == 0) {
        double *rc = region<double>(a.ws, L.rowconst) + int64_t(row) * 4;
        rc[0] = 1.0;
        rc[1] = e;
        rc[2] = scale;
        rc[3] = 0.0;
    }
    // the transform returns 2 X: |2 X|^2 scale^2 / 4 (exact scalings)
    const real scale2 = static_cast<real>(scale * scale) * real(0.25);

    float *bark = region<float>(a.ws, L.bark) + int64_t(row) * L.frames * kBands;
    cplx<real> *buf = fftbuf[wave];
    real *power_buf = reinterpret_cast<real *>(buf);
    // kLean reads the twiddles per pass from LDS; otherwise they stay in registers
    using TW = typename std::conditional<kLean, LdsTwiddles<real>, Twiddles<real>>::type;
    TW tw;
    if constexpr (kLean) {
        for (int i = threadIdx.x; i < kNfft; i += kWave * kWaves) {
            if (i < kPassTwiddles) lds_pass[i] = StagedTwiddles<real>::pass(t)[i];
            if (i < kHalf) lds_tw512[i] = StagedTwiddles<real>::fold(t)[i];
            lds_win[i] = t.window[i];
        }
        __syncthreads();
        tw = TW{lds_pass, lds_tw512, lane};
    } else {
        tw.load_staged(StagedTwiddles<real>::pass(t), StagedTwiddles<real>::fold(t), lane);
    }
    float win[8];
    if constexpr (!kLean) {
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            win[2 * r] = t.window[2 * (lane + 64 * r)];
            win[2 * r + 1] = t.window[2 * (lane + 64 * r) + 1];
        }
    }
    const int band_lo = lane < kBands ? t.band_start[lane] : 0;
    const int band_hi = lane < kBands ? t.band_end[lane] : 0;
    const double corr = lane < kBands ? t.corr[lane] : 0.0;
    const double th100 = lane < kBands ? 100.0 * t.threshs[lane] : 0.0;

    for (int q = 0; q < kPerWave; ++q) {
        const int local = (wave % kSideWaves) * kPerWave + q;
        const int64_t frame = t0 + local;
        if (frame >= L.frames) break;
        // the next frame's samples load while this one is transformed
        float nxt[8];
        if constexpr (!kLean) {
            const int64_t fn = frame + 1 < L.frames ? frame + 1 : frame;
            load_frame(p, fn * kHop, L.len, lane, nxt);
        } else {
            if (q > 0) load_frame(p, frame * kHop, L.len, lane, cur);
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                win[2 * r] = lds_win[2 * (lane + 64 * r)];
                win[2 * r + 1] = lds_win[2 * (lane + 64 * r) + 1];
            }
        }
        auto u = [&](int k) -> real {
            // k = 2 (lane + 64 r) + {0, 1}: sample and window value at index 2 r + {0, 1}
            const int i = 2 * (k >> 7) + (k & 1);
            return static_cast<real>(cur[i]) * static_cast<real>(win[i]);
        };
        cplx<real> x[4];
        frame_spectrum<real, true>(u, x, buf, tw, lane);
        if constexpr (!kLean) {
#pragma unroll
            for (int i = 0; i < 8; ++i) cur[i] = nxt[i];
        }
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int fbin = lane + 64 * r;
            power_buf[fbin] =
                fbin == 0 ? real(0) : fmadd(x[r].re, x[r].re, x[r].im * x[r].im) * scale2;
        }
        wave_lds_fence();
        const double acc = band_power(power_buf, lane, band_lo, band_hi);
        double val = 0.0;
        if (lane < kBands) {
            const float v = static_cast<float>(acc * corr);
            bark[frame * kBands + lane] = v;
            barks[side][local][lane] = v;
            val = v;
        }
        wave_lds_fence();
        if (side == 0) {
            // silent frame: audible (> 100 th) energy of the reference below 1e7
            const double aud = lane < kBands && val > th100 ? val : 0.0;
            const double total = wave_sum(aud);
            if (lane == 0) {
                const float k = total >= 1e7 ? 1.0f : 0.0f;
                keepflag[local] = k;
                region<float>(a.ws, L.keep)[int64_t(item) * L.frames + frame] = k;
            }
        }
    }
    __syncthreads();

    // band partial sums of the audible, non silent frames of this tile
    if (wave < 2 && lane < kBands) {
        const double th100 = 100.0 * t.threshs[lane];
        double acc = 0.0;
#pragma unroll
        for (int local = 0; local < kTile; ++local) {
            const double v = barks[wave][local][lane];
            if (t0 + local < L.frames && keepflag[local] != 0.0f && v > th100) acc += v;
        }
        double *dst = region<double>(a.ws, wave == 0 ? L.bandref : L.banddeg);
        dst[(int64_t(item) * L.ntile + tile) * kBands + lane] = acc;
    }
}

// ---------------------------------------------------------------------------
// 3b. per item band totals (items of more than kTotalsTiles chain tiles)
// ---------------------------------------------------------------------------

// Sums over all tiles of an item of the per tile band partials: forward
// (kArrays 2), the audible band powers of both signals (bandref, banddeg ->
// bandtot), read by the chain forward; backward (kArrays 1), the band
// gradient partials (grpart -> gradtot), read by the STFT backward.  Each sum
// runs in the order the reading kernel would take it itself: kSlices slices
// of tiles v, v + kSlices, ... (in tile order), then the slices in order, so
// the totals are those bits.  One workgroup per item, wavefront v a slice,
// a lane a band.
template <int kSlices, int kArrays>
__global__ void __launch_bounds__(kWave *kSlices) band_totals_kernel(PipeArgs a) {
    __shared__ double part[kArrays][kSlices][kBands];
    const PipeLayout &L = a.L;
    const int item = blockIdx.x;
    const int wave = wave_index();
    const int lane = threadIdx.x % kWave;
    const double *src[kArrays];
    double *dst;
    if constexpr (kArrays == 2) {
        src[0] = region<double>(a.ws, L.bandref) + int64_t(item) * L.ntile * kBands;
        src[kArrays - 1] = region<double>(a.ws, L.banddeg) + int64_t(item) * L.ntile * kBands;
        dst = region<double>(a.ws, L.bandtot) + int64_t(item) * 2 * kBands;
    } else {
        src[0] = region<double>(a.bw, L.grpart) + int64_t(item) * L.ntile * kBands;
        dst = region<double>(a.bw, L.gradtot) + int64_t(item) * kBands;
    }
    if (lane < kBands) {
        // the slice's tiles wave, wave + kSlices, ... of every array, with the
        // loads of all arrays in flight together, 8 per array at a time
        const double *ptr[kArrays];
        int cnt[kArrays];
        const int n = L.ntile > wave ? static_cast<int>((L.ntile - 1 - wave) / kSlices) + 1 : 0;
#pragma unroll
        for (int k = 0; k < kArrays; ++k) {
            ptr[k] = src[k] + int64_t(wave) * kBands + lane;
            cnt[k] = n;
        }
        double sums[kArrays];
        strided_sums<kArrays, 8>(ptr, cnt, int64_t(kSlices) * kBands, sums);
#pragma unroll
        for (int k = 0; k < kArrays; ++k) part[k][wave][lane] = sums[k];
    }
    __syncthreads();
    if (wave == 0 && lane < kBands) {
#pragma unroll
        for (int k = 0; k < kArrays; ++k) {
            double sum = 0.0;
            for (int v = 0; v < kSlices; ++v) sum += part[k][v][lane];
            dst[k * kBands + lane] = sum;
        }
    }
}

// ---------------------------------------------------------------------------
// 4. chain forward per (item, 16 frames)
// ---------------------------------------------------------------------------

struct BandConsts {
    double th, inv2th, e, ls, w;
};

__device__ __forceinline__ BandConsts band_consts(const ModelTable &t, int band, int nb) {
    BandConsts c{1.0, 0.5, 1.0, 0.0, 0.0};
    if (band < nb) {
        c.th = t.threshs[band];
        c.inv2th = 0.5 / c.th;
        c.e = t.exps[band];
        c.ls = t.loud_scale[band];
        c.w = t.width[band];
    }
    return c;
}

// The chain kernels run a 16 frame tile with kWaves wavefronts of kTile /
// kWaves frames each: one frame per wavefront when the grid has about one
// workgroup per CU (latency bound), more frames per wavefront for larger
// batches (throughput bound; more work per wave in flight).  Every sum that
// crosses wavefronts is taken in the same per frame / per slice order for
// any kWaves, so the results do not depend on the choice.
constexpr int kChainSlices = 16;  // fixed split of the band partial sums

template <int kWaves, int kBPL>
__global__ void __launch_bounds__(kWave *kWaves) chain_fwd_kernel(PipeArgs a) {
    constexpr int kPer = kTile / kWaves;  // frames per wavefront
    __shared__ double part[2][kChainSlices][kWave * kBPL];
    __shared__ double red_lds[kWaves][wave_sums_lds_doubles<2 * (kPer + 1)>()];

    const ModelTable &t = *a.tab;
    const PipeLayout &L = a.L;
    const int wave = wave_index();
    const int lane = threadIdx.x % kWave;
    const int nb = L.nb;  // bands: band lane + kWave k is slot k of a lane
    const int item = blockIdx.x / L.ntile;
    const int tile = blockIdx.x - item * L.ntile;
    const int t0 = tile * kTile;
    const double frames_f = static_cast<double>(L.frames);
    const int64_t f0 = t0 + wave * kPer;  // first frame of this wavefront

    // Bark values of frames f0 - 1 .. f0 + kPer - 1, loaded up front (indices
    // clamped into the array; out of range frames and bands are masked later)
    float R[kBPL][kPer + 1], G[kBPL][kPer + 1];
    {
        const float *bref = a.bark_ref + int64_t(item) * L.frames * nb;
        const float *bdeg = a.bark_deg + int64_t(item) * L.frames * nb;
#pragma unroll
        for (int k = 0; k < kBPL; ++k) {
            const int band = lane + kWave * k < nb ? lane + kWave * k : nb - 1;
#pragma unroll
            for (int q = 0; q <= kPer; ++q) {
                int64_t frame = f0 - 1 + q;
                frame = frame < 0 ? 0 : (frame >= L.frames ? L.frames - 1 : frame);
                R[k][q] = bref[frame * nb + band];
                G[k][q] = bdeg[frame * nb + band];
            }
        }
    }

    // band constants and the uniform reciprocals, requested before the barrier
    // (which would hold back loads issued after it)
    BandConsts c[kBPL];
#pragma unroll
    for (int k = 0; k < kBPL; ++k) c[k] = band_consts(t, lane + kWave * k, nb);
    const double W = t.total_width;
    const double inv_sqrt_w = 1.0 / sqrt(W);
    const double inv_w = 1.0 / W;

    // mean band powers over all frames of the item: slice v sums the band
    // partials of tiles v, v + kChainSlices, ...; the slices are then added in
    // order, the same order in every workgroup (wavefront w takes slices w,
    // w + kWaves, ...).  Items of many tiles read the sums band_totals_kernel
    // took in that order.
    if (!L.totals) {
        const double *pr = region<double>(a.ws, L.bandref) + int64_t(item) * L.ntile * nb;
        const double *pd = region<double>(a.ws, L.banddeg) + int64_t(item) * L.ntile * nb;
        constexpr int kMine = kChainSlices / kWaves;  // slices per wavefront
        static_assert(kMine * kWaves == kChainSlices, "slices split evenly over the wavefronts");
#pragma unroll
        for (int k = 0; k < kBPL; ++k) {
            const int band = lane + kWave * k;
            if (band < nb) {
                // tile_partial of both arrays for each of the wavefront's slices,
                // with all their loads in flight together
                const double *ptr[2 * kMine];
                int cnt[2 * kMine];
#pragma unroll
                for (int j = 0; j < kMine; ++j) {
                    const int v = wave + j * kWaves;
                    const int n = L.ntile > v ? static_cast<int>((L.ntile - 1 - v) / kChainSlices) + 1 : 0;
                    ptr[2 * j] = pr + int64_t(v) * nb + band;
                    ptr[2 * j + 1] = pd + int64_t(v) * nb + band;
                    cnt[2 * j] = cnt[2 * j + 1] = n;
                }
                double sums[2 * kMine];
                strided_sums(ptr, cnt, int64_t(kChainSlices) * nb, sums);
#pragma unroll
                for (int j = 0; j < kMine; ++j) {
                    part[0][wave + j * kWaves][band] = sums[2 * j];
                    part[1][wave + j * kWaves][band] = sums[2 * j + 1];
                }
            }
        }
    }
    __syncthreads();

    bool live[kBPL];
    double r[kBPL];
#pragma unroll
    for (int k = 0; k < kBPL; ++k) {
        const int band = lane + kWave * k;
        live[k] = band < nb;
        r[k] = 0.0;
        if (live[k]) {
            double sr = 0.0, sd = 0.0;
            if (L.totals) {
                const double *tot = region<double>(a.ws, L.bandtot) + int64_t(item) * 2 * nb;
                sr = tot[band];
                sd = tot[nb + band];
            } else {
                for (int v = 0; v < kChainSlices; ++v) {
                    sr += part[0][v][band];
                    sd += part[1][v][band];
                }
            }
            const double mref = sr / frames_f;
            const double mdeg = sd / frames_f;
            const double ratio = (mdeg + 1000.0) / (mref + 1000.0);
            r[k] = fmin(fmax(ratio, 0.01), 100.0);
            if (tile == 0 && wave == 0) {
                band_array(a, kR)[item * nb + band] = r[k];
                band_array(a, kRatio)[item * nb + band] = ratio;
                band_array(a, kMref)[item * nb + band] = mref;
            }
        }
    }
    // per frame totals of the audible energies; slot q is frame f0 - 1 + q
    // (a lane adds its bands, then the lanes are summed, all slots together)
    double *red = red_lds[wave];
    double tv[2 * (kPer + 1)];
#pragma unroll
    for (int q = 0; q <= kPer; ++q) {
        const int64_t frame = f0 - 1 + q;
        const bool fok = frame >= 0 && frame < L.frames;
        double ar = 0.0, ad = 0.0;
#pragma unroll
        for (int k = 0; k < kBPL; ++k) {
            const bool ok = live[k] && fok;
            const double er = r[k] * static_cast<double>(R[k][q]);
            const double g = G[k][q];
            const double xr = ok && er > c[k].th ? er : 0.0;
            const double xd = ok && g > c[k].th ? g : 0.0;
            ar = k == 0 ? xr : ar + xr;  // a lane's first band starts the sum
            ad = k == 0 ? xd : ad + xd;
        }
        tv[2 * q] = ar;
        tv[2 * q + 1] = ad;
    }
    // totals of slot q (taer, tad) in lanes 8 q .. 8 q + 3 and 8 q + 4 .. 8 q + 7
    const double tsum = wave_sums_lds(tv, red, lane);

    // per frame quantities of the wavefront's frames f0 - 1 .. f0 + kPer - 1,
    // frame slot q in lane q, read back per frame: the unsmoothed frame ratio
    // (taer + 5e3) / (tad + 5e3), h = ((taer + 1e5) / 1e7)^0.04 and 1 / h
    const int slot = lane <= kPer ? lane : 0;
    const double t_lane = shfl(tsum, 8 * slot);
    const double d_lane = shfl(tsum, 8 * slot + 4);
    const double fpr0_lane = (t_lane + 5e3) / (d_lane + 5e3);
    const double h_lane = exp_chain(0.04 * log_ratio_refined(t_lane + 1e5, 1e7));
    const double inv_h_lane = 1.0 / h_lane;
    const double fpr0_prev_lane = wave_shift_up(fpr0_lane);  // slot q - 1 in lane q

    double vy[2 * kPer];  // per lane terms of the weighted norms of each frame
#pragma unroll
    for (int q = 0; q < kPer; ++q) {
        vy[2 * q] = vy[2 * q + 1] = 0.0;
        const int64_t frame = f0 + q;
        if (frame >= L.frames) continue;
        const double fpr0 = read_lane(fpr0_lane, q + 1);
        const double fpr1 = frame > 0 ? fpr0 * 0.8 + read_lane(fpr0_lane, q) * 0.2 : fpr0;
        const double fpr = fmin(fmax(fpr1, 3e-4), 5.0);

        double v2 = 0.0, ya = 0.0;
#pragma unroll
        for (int k = 0; k < kBPL; ++k) {
            double xv = 0.0, xa = 0.0;
            if (live[k]) {
                const BandConsts &ck = c[k];
                const double er = r[k] * static_cast<double>(R[k][q + 1]);
                const double ed = fpr * static_cast<double>(G[k][q + 1]);
                const double lr = loudness(er, ck.th, ck.inv2th, ck.e, ck.ls);
                const double ld = loudness(ed, ck.th, ck.inv2th, ck.e, ck.ls);
                const double u = ld - lr;
                const double z = fabs(u) - 0.25 * fmin(ld, lr);
                const double dist = sgn(u) * fmax(z, 0.0);
                const double asc_raw = asymmetry(ed, er);
                const double asc = asc_raw < 3.0 ? 0.0 : fmin(asc_raw, 12.0);
                if (L.loud_store) {
                    const int64_t o = (int64_t(item) * L.frames + frame) * nb + lane + kWave * k;
                    const double asc_s = asc_raw < 3.0 ? 0.0 : (asc_raw <= 12.0 ? asc_raw : -12.0);
                    chain_terms(a)[o] = {static_cast<float>(dist), static_cast<float>(asc_s),
                                         loudness_slope(er, lr, ck.th, ck.e, ck.ls),
                                         loudness_slope(ed, ld, ck.th, ck.e, ck.ls)};
                }
                if (lane + kWave * k >= 1) {
                    const double v = ck.w * dist * inv_sqrt_w;
                    xv = v * v;
                    xa = fabs(ck.w * (dist * asc) * inv_w);
                }
            }
            v2 = k == 0 ? xv : v2 + xv;
            ya = k == 0 ? xa : ya + xa;
        }
        vy[2 * q] = v2;
        vy[2 * q + 1] = ya;
    }
    // the norms of frame q in lanes 8 q .. 8 q + 3 (squares) and 8 q + 4 .. + 7
    const double nsum = wave_sums_lds(vy, red, lane);
    const int fq = lane >= 1 && lane <= kPer ? lane - 1 : 0;
    const double v2_lane = shfl(nsum, 8 * fq), ya_lane = shfl(nsum, 8 * fq + 4);

    // the chain state of frame f0 + l - 1, written by lane l = 1 .. kPer
    const int64_t frame_l = f0 + lane - 1;
    if (lane >= 1 && lane <= kPer && frame_l < L.frames) {
        const double fpr1 = frame_l > 0 ? fpr0_lane * 0.8 + fpr0_prev_lane * 0.2 : fpr0_lane;
        const double symm_raw = W * sqrt(v2_lane);
        const double asymm_raw = W * ya_lane;
        const int64_t o = int64_t(item) * L.frames + frame_l;
        frame_array(a, kTaer)[o] = t_lane;
        frame_array(a, kTad)[o] = d_lane;
        frame_array(a, kFpr0)[o] = fpr0_lane;
        frame_array(a, kFpr1)[o] = fpr1;
        frame_array(a, kH)[o] = h_lane;
        frame_array(a, kSymmRaw)[o] = symm_raw;
        frame_array(a, kAsymmRaw)[o] = asymm_raw;
        frame_array(a, kSymm)[o] = fmin(fmax(symm_raw, 1e-20) * inv_h_lane, 45.0);
        frame_array(a, kAsymm)[o] = fmin(fmax(asymm_raw, 1e-20) * inv_h_lane, 45.0);
    }
}

// ---------------------------------------------------------------------------
// 5. overlapping sums, distances, MOS and loss, one workgroup per item
// ---------------------------------------------------------------------------

constexpr int kFinalMaxThreads = 1024;

// Threads per workgroup of chain_final_kernel: one PSQM window per thread up to
// 1024 windows (a second window per thread doubles the kernel's latency), in
// whole wavefronts (a single one, at most 64 windows, needs no barrier wait on
// others).
static unsigned final_threads(int64_t nwin) {
    const int64_t waves = (nwin + kWave - 1) / kWave;
    return static_cast<unsigned>(kWave * (waves < 1 ? 1 : (waves > 16 ? 16 : waves)));
}

// both frame arrays (symmetric, asymmetric) in the same pass over the PSQM
// windows, so that their loads, powers and block sums overlap; each sum is
// per wave (wave_sum), then over the waves in order
__global__ void __launch_bounds__(kFinalMaxThreads) chain_final_kernel(PipeArgs a) {
    __shared__ double scratch[2][kFinalMaxThreads / kWave];
    const int waves = static_cast<int>(blockDim.x) / kWave;
    const PipeLayout &L = a.L;
    const int item = blockIdx.x;
    const double *s0 = frame_array(a, kSymm) + int64_t(item) * L.frames;
    const double *s1 = frame_array(a, kAsymm) + int64_t(item) * L.frames;
    double *psqm0 = region<double>(a.ws, L.psqm) + int64_t(item) * L.nwin;
    double *psqm1 = psqm0 + L.batch * L.nwin;
    double acc0 = 0.0, acc1 = 0.0;
    for (int64_t l = threadIdx.x; l < L.nwin; l += blockDim.x) {
        double m0 = 0.0, m1 = 0.0;
        for (int j = 0; j < kWin; ++j) {
            const double v0 = s0[l * kStride + j], v1 = s1[l * kStride + j];
            const double q0 = v0 * v0, q1 = v1 * v1;
            m0 += q0 * q0 * q0;
            m1 += q1 * q1 * q1;
        }
        // x^(1/6) as sqrt(cbrt(x)): about the same rounding as pow(x, 1 / 6.0)
        // (whose exponent is itself rounded), at a fraction of its cost
        const double pl0 = sqrt(cbrt(m0 / kWin)), pl1 = sqrt(cbrt(m1 / kWin));
        psqm0[l] = pl0;
        psqm1[l] = pl1;
        acc0 += pl0 * pl0;
        acc1 += pl1 * pl1;
    }
    acc0 = wave_sum(acc0);
    acc1 = wave_sum(acc1);
    const int wave = wave_index();
    if ((threadIdx.x % kWave) == 0) {
        scratch[0][wave] = acc0;
        scratch[1][wave] = acc1;
    }
    __syncthreads();
    double d[2] = {0.0, 0.0};
    for (int i = 0; i < waves; ++i) {
        d[0] += scratch[0][i];
        d[1] += scratch[1][i];
    }
    d[0] = sqrt(d[0] / static_cast<double>(L.nwin));
    d[1] = sqrt(d[1] / static_cast<double>(L.nwin));
    if (threadIdx.x == 0) {
        double *dist = region<double>(a.ws, L.dist) + int64_t(item) * 2;
        dist[0] = d[0];
        dist[1] = d[1];
        const double inner = 4.5 - 0.1 * d[0] - 0.0309 * d[1];
        a.d_symm[item] = static_cast<float>(d[0]);
        a.d_asymm[item] = static_cast<float>(d[1]);
        if (a.mos) a.mos[item] = static_cast<float>(0.999 + 4.0 / (1.0 + exp(-1.3669 * inner + 3.8224)));
        if (a.loss) a.loss[item] = static_cast<float>(a.factor * (0.1 * d[0] + 0.0309 * d[1]));
    }
}

// ---------------------------------------------------------------------------
// 6. chain backward per (item, 16 frames)
// ---------------------------------------------------------------------------

// PSQM windows that touch the frames t0 .. t0 + kTile of one chain tile:
// l in [t0 / kStride - 1, (t0 + kTile) / kStride], at most kPsqmSlots of them.
constexpr int kPsqmSlots = (kTile + kStride - 1) / kStride + 2;

// d d / d s_t of d = sqrt(mean_l psqm_l^2), psqm_l = (mean_{j<20} s_{10 l + j}^6)^(1/6);
// pl[i] holds psqm_{lbase + i}
// (inv_nd = 1 / (nwin d))
__device__ __forceinline__ double psqm_adjoint(const PipeLayout &L, const double *pl,
                                               int64_t lbase, double d, double inv_nd, double s,
                                               int64_t frame) {
    if (!(d > 0.0)) return 0.0;
    double acc = 0.0;
    const int64_t hi = frame / kStride;
    for (int64_t l = hi - 1; l <= hi; ++l) {
        if (l < 0 || l >= L.nwin || frame >= l * kStride + kWin) continue;
        const double p = pl[l - lbase];
        if (!(p > 0.0)) continue;
        const double ratio = s / p;
        const double r2 = ratio * ratio;
        acc += p * inv_nd * (r2 * r2 * ratio) * (1.0 / kWin);
    }
    return acc;
}

// the 4 wavefront single band variant (large grids) is held to 128 VGPRs, four
// workgroups per CU
template <int kWaves, int kBPL>
__global__ void __launch_bounds__(kWave *kWaves, kWaves == 4 && kBPL == 1 ? 4 : 1)
    chain_bwd_kernel(PipeArgs a) {
    constexpr int kPer = kTile / kWaves;
    constexpr int kSlots = kTile + 1;  // the tile's frames and the next one
    constexpr int kLaneBands = kWave * kBPL;
    __shared__ double rs[kLaneBands];
    __shared__ double fr[kFrameArrays][kSlots];
    __shared__ double pl[2][kPsqmSlots];
    __shared__ double gfpr[kSlots], gh[kSlots];
    __shared__ double part[kTile][kLaneBands];  // per frame band partials
    __shared__ double red_lds[kWaves][wave_sums_lds_doubles<kPer + 1>()];

    const ModelTable &t = *a.tab;
    const PipeLayout &L = a.L;
    const int nb = L.nb;  // bands: band lane + kWave k is slot k of a lane
    const int item = blockIdx.x / L.ntile;
    const int tile = blockIdx.x - item * L.ntile;
    const int t0 = tile * kTile;
    const int wave = wave_index();
    const int lane = threadIdx.x % kWave;
    bool live[kBPL];
#pragma unroll
    for (int k = 0; k < kBPL; ++k) live[k] = lane + kWave * k < nb;
    const int64_t fo = int64_t(item) * L.frames;
    const int64_t lbase = t0 / kStride - 1;

    // Bark values of this wavefront's frames (slot q = local frame wave kPer
    // + q) and, with one frame per wavefront, the forward's per (frame, band)
    // terms too: requested before the barrier, which would hold back loads
    // issued after it.  The variants of more frames per wavefront load the
    // terms where they use them: held in registers they would cost a
    // wavefront per SIMD.
    constexpr bool kEarlyTerms = kPer == 1;
    float R[kBPL][kPer + 1], G[kBPL][kPer + 1];
    ChainTerms cts[kEarlyTerms ? kBPL : 1][kEarlyTerms ? kPer + 1 : 1];
    {
        const float *bref = a.bark_ref + int64_t(item) * L.frames * nb;
        const float *bdeg = a.bark_deg + int64_t(item) * L.frames * nb;
        const ChainTerms *terms = chain_terms(a);
#pragma unroll
        for (int k = 0; k < kBPL; ++k) {
            const int band = live[k] ? lane + kWave * k : nb - 1;
#pragma unroll
            for (int q = 0; q <= kPer; ++q) {
                const int64_t frame = t0 + wave * kPer + q;
                const int64_t fc = frame < L.frames ? frame : L.frames - 1;
                R[k][q] = bref[fc * nb + band];
                G[k][q] = bdeg[fc * nb + band];
                if constexpr (kEarlyTerms) cts[k][q] = terms[(fo + fc) * nb + band];
            }
        }
    }

    // the tile's per frame chain state and PSQM windows, one load per thread
    if (threadIdx.x < kFrameArrays * kSlots) {
        const int which = threadIdx.x / kSlots;
        const int q = threadIdx.x - which * kSlots;
        const int64_t frame = t0 + q < L.frames ? t0 + q : L.frames - 1;
        fr[which][q] = frame_array(a, which)[fo + frame];
    } else if (threadIdx.x >= 192 && threadIdx.x < 192 + 2 * kPsqmSlots) {
        const int side = (threadIdx.x - 192) / kPsqmSlots;
        const int i = threadIdx.x - 192 - side * kPsqmSlots;
        int64_t l = lbase + i;
        l = l < 0 ? 0 : (l >= L.nwin ? L.nwin - 1 : l);
        pl[side][i] = region<double>(a.ws, L.psqm)[(int64_t(side) * L.batch + item) * L.nwin + l];
    }
    if (wave == 0) {
#pragma unroll
        for (int k = 0; k < kBPL; ++k) {
            if (live[k]) rs[lane + kWave * k] = band_array(a, kR)[item * nb + lane + kWave * k];
        }
    }
    // band constants, requested before the barrier (which would hold them back)
    BandConsts c[kBPL];
#pragma unroll
    for (int k = 0; k < kBPL; ++k) c[k] = band_consts(t, lane + kWave * k, nb);
    const double W = t.total_width;

    // upstream gradients of the two distances, MOS and loss folded in
    const double *dist = region<double>(a.ws, L.dist) + int64_t(item) * 2;
    const double ds = dist[0], da = dist[1];
    const double inv_nds = ds > 0.0 ? 1.0 / (static_cast<double>(L.nwin) * ds) : 0.0;
    const double inv_nda = da > 0.0 ? 1.0 / (static_cast<double>(L.nwin) * da) : 0.0;
    double gds = a.g_symm ? a.g_symm[item] : 0.0;
    double gda = a.g_asymm ? a.g_asymm[item] : 0.0;
    if (a.g_loss) {
        gds += a.g_loss[item] * a.factor * 0.1;
        gda += a.g_loss[item] * a.factor * 0.0309;
    }
    if (a.g_mos) {
        const double inner = 4.5 - 0.1 * ds - 0.0309 * da;
        const double ex = exp(-1.3669 * inner + 3.8224);
        const double dmos = 4.0 * 1.3669 * ex / ((1.0 + ex) * (1.0 + ex));
        gds += a.g_mos[item] * dmos * -0.1;
        gda += a.g_mos[item] * dmos * -0.0309;
    }
    __syncthreads();

    double r[kBPL];
#pragma unroll
    for (int k = 0; k < kBPL; ++k) r[k] = live[k] ? rs[lane + kWave * k] : 0.0;

    // phase 1: adjoint of the per frame distances down to equ_ref / equ_deg
    double g_er[kBPL][kPer + 1], g_ed[kBPL][kPer + 1];
    double gfv[kPer + 1], ghh[kPer + 1];  // per lane d/d fpr terms, d/d h of each slot
    const int nmine = wave == kWaves - 1 ? kPer + 1 : kPer;
#pragma unroll
    for (int q = 0; q <= kPer; ++q) {
        const int local = wave * kPer + q;
        const int64_t frame = t0 + local;
#pragma unroll
        for (int k = 0; k < kBPL; ++k) g_er[k][q] = g_ed[k][q] = 0.0;
        gfv[q] = ghh[q] = 0.0;
        if (q >= nmine || frame >= L.frames) continue;

        const double s_sy = fr[kSymm][local];
        const double s_as = fr[kAsymm][local];
        const double g_sy = gds * psqm_adjoint(L, pl[0], lbase, ds, inv_nds, s_sy, frame);
        const double g_as = gda * psqm_adjoint(L, pl[1], lbase, da, inv_nda, s_as, frame);
        const double raw_s = fr[kSymmRaw][local];
        const double raw_a = fr[kAsymmRaw][local];
        const double h = fr[kH][local];
        const double inv_h = 1.0 / h;  // the forward's clamp used the same product
        const double pre_s = fmax(raw_s, 1e-20), pre_a = fmax(raw_a, 1e-20);
        const double g_ps = pre_s * inv_h <= 45.0 ? g_sy : 0.0;
        const double g_pa = pre_a * inv_h <= 45.0 ? g_as : 0.0;
        const double g_hh = -(g_ps * pre_s + g_pa * pre_a) * (inv_h * inv_h);
        const double g_rs = raw_s >= 1e-20 ? g_ps * inv_h : 0.0;
        const double g_ra = raw_a >= 1e-20 ? g_pa * inv_h : 0.0;
        const double inv_raw_s = raw_s > 0.0 ? 1.0 / raw_s : 0.0;
        const double fpr = fmin(fmax(fr[kFpr1][local], 3e-4), 5.0);

        double gf = 0.0;
#pragma unroll
        for (int k = 0; k < kBPL; ++k) {
            double my_er = 0.0, my_ed = 0.0, xg = 0.0;
            if (live[k]) {
                const BandConsts &ck = c[k];
                const double Rq = R[k][q], Gq = G[k][q];
                const double er = r[k] * Rq, ed = fpr * Gq;
                // the forward's terms of this (frame, band)
                const ChainTerms ct = kEarlyTerms
                                          ? cts[kEarlyTerms ? k : 0][kEarlyTerms ? q : 0]
                                          : chain_terms(a)[(fo + frame) * nb + lane + kWave * k];
                const double dst = ct.dist;
                const double asc = fabs(static_cast<double>(ct.asc));
                const double su = sgn(dst);

                double g_dist = 0.0, g_asc = 0.0;
                if (lane + kWave * k >= 1) {
                    if (raw_s > 0.0) g_dist = g_rs * W * ck.w * ck.w * dst * inv_raw_s;
                    const double gy = g_ra * ck.w * sgn(dst * asc);
                    g_dist += gy * asc;
                    g_asc = gy * dst;
                }
                // outside the dead zone (dst != 0) the smaller loudness is the
                // reference's where u > 0 and the degraded one's where u < 0;
                // inside it g_dist is 0 and so are g_u and g_min
                const double g_u = g_dist * su * su;
                const double g_min = -0.25 * g_dist * su;
                const double g_ld = g_u + (su < 0.0 ? g_min : 0.0);
                const double g_lr = -g_u + (su > 0.0 ? g_min : 0.0);
                my_er = g_lr * static_cast<double>(ct.sr);
                my_ed = g_ld * static_cast<double>(ct.sd);
                if (ct.asc > 0.0f) {
                    const double g_log = g_asc * 1.2 * asc;  // d asc / d log(ratio)
                    my_ed += g_log / (ed + 50.0);
                    my_er -= g_log / (er + 50.0);
                }
                xg = my_ed * Gq;
            }
            g_er[k][q] = my_er;
            g_ed[k][q] = my_ed;
            gf = k == 0 ? xg : gf + xg;
        }
        gfv[q] = gf;
        ghh[q] = g_hh;
    }
    {
        // the lane sums of all slots together: slot q's in lanes 4 q .. 4 q + 3
        const double gsum = wave_sums_lds(gfv, red_lds[wave], lane);
#pragma unroll
        for (int q = 0; q <= kPer; ++q) {
            const int local = wave * kPer + q;
            if (q < nmine && t0 + local < L.frames && lane == 4 * q) {
                gfpr[local] = gsum;
                gh[local] = ghh[q];
            }
        }
    }
    __syncthreads();

    // phase 2: frame power ratio, h and the total audible energies; the
    // band partials of d/dr are kept per frame and added in frame order
#pragma unroll
    for (int q = 0; q < kPer; ++q) {
#pragma unroll
        for (int k = 0; k < kBPL; ++k) {
            if (live[k]) part[wave * kPer + q][lane + kWave * k] = 0.0;
        }
    }
#pragma unroll
    for (int q = 0; q < kPer; ++q) {
        const int local = wave * kPer + q;
        const int64_t frame = t0 + local;
        if (frame >= L.frames) break;
        const double f1 = fr[kFpr1][local];
        const double g1 = (f1 >= 3e-4 && f1 <= 5.0) ? gfpr[local] : 0.0;
        double g1n = 0.0;
        if (frame + 1 < L.frames) {
            const double f1n = fr[kFpr1][local + 1];
            g1n = (f1n >= 3e-4 && f1n <= 5.0) ? gfpr[local + 1] : 0.0;
        }
        const double g0 = (frame == 0 ? g1 : 0.8 * g1) + 0.2 * g1n;
        const double taer = fr[kTaer][local];
        const double tad = fr[kTad][local];
        const double fpr0 = fr[kFpr0][local];
        const double h = fr[kH][local];
        const double inv_tad = 1.0 / (tad + 5e3);
        const double g_taer = g0 * inv_tad + gh[local] * 0.04 * h / (taer + 1e5);
        const double g_tad = -g0 * fpr0 * inv_tad;
        const double fpr = fmin(fmax(f1, 3e-4), 5.0);
#pragma unroll
        for (int k = 0; k < kBPL; ++k) {
            if (!live[k]) continue;
            const int band = lane + kWave * k;
            const double Rq = R[k][q], Gq = G[k][q];
            double ger = g_er[k][q];
            if (r[k] * Rq > c[k].th) ger += g_taer;
            const double ged = g_ed[k][q] * fpr + (Gq > c[k].th ? g_tad : 0.0);
            a.gbark_ref[(int64_t(item) * L.frames + frame) * nb + band] = static_cast<float>(ger * r[k]);
            a.gbark_deg[(int64_t(item) * L.frames + frame) * nb + band] = static_cast<float>(ged);
            part[local][band] = ger * Rq;
        }
    }
    __syncthreads();
    if (wave == 0) {
#pragma unroll
        for (int k = 0; k < kBPL; ++k) {
            if (!live[k]) continue;
            const int band = lane + kWave * k;
            double s = 0.0;
            for (int f = 0; f < kTile; ++f) s += part[f][band];
            region<double>(a.bw, L.grpart)[(int64_t(item) * L.ntile + tile) * nb + band] = s;
        }
    }
}

// ---------------------------------------------------------------------------
// 7. STFT backward per (grad row, kW kFPW - 1 hop blocks)
// ---------------------------------------------------------------------------

// kW wavefronts of kFPW frames each: wavefront w transforms the workgroup's
// frames w, w + kW, ...  Small grids take one frame per wavefront and nine
// wavefronts (at c2 the 504 workgroups of 9 all fit on the chip at once, two
// per CU, where 576 of 8 do not: 10.2 against 11.4 us; 448 of 10, 10.7 us);
// large ones two frames per wavefront and eight wavefronts,
// which halves the per workgroup table staging and band sums per frame and
// the frames shared by two workgroups.  Every sum is taken in an order that
// does not depend on the variant: the band gradient totals over kGradSlices
// slices of tiles (the first kGradSlices wavefronts take one each), and the
// partials of S = sum dL/dp . p per hop block (one wavefront's lanes over its
// 256 samples), so an item gets the same bits in any batch.
constexpr int kGradSlices = kBwdWaves;

template <typename real, int kFPW, int kW>
__global__ void __launch_bounds__(kWave *kW, kFPW == 2 ? 4 : 5) stft_bwd_kernel(PipeArgs a) {
#pragma clang fp contract(off)  // the same bits in both variants (spectral.hpp)
    static_assert(kW >= kGradSlices, "a wavefront per slice of the band gradient totals");
    constexpr int kFrames = kW * kFPW;  // frames per workgroup
    constexpr int kHops = kFrames - 1;         // output hop blocks per workgroup
    __shared__ cplx<real> fftbuf[kW][kHalf];
    __shared__ float contrib[kFrames][kNfft];
    __shared__ double gpart[kGradSlices][kBands];
    __shared__ float gband[kW][kBands];
    // the twiddle tables, window and bin-to-band map, staged once per
    // workgroup (both FFTs of every frame read them)
    using T2 = typename Vec2<real>::type;
    __shared__ T2 lds_pass[kPassTwiddles], lds_tw512[kHalf];
    __shared__ float lds_win[kNfft];
    __shared__ int lds_bin_band[kHalf];

    const ModelTable &t = *a.tab;
    const PipeLayout &L = a.L;
    const int i = blockIdx.x / L.nhoptile;       // gradient row index
    const int ht = blockIdx.x - i * L.nhoptile;
    const int row = L.row0 + i;                  // stacked row
    const int item = row % L.batch;
    const bool is_ref = row < L.batch;
    const int wave = wave_index();
    const int lane = threadIdx.x % kWave;
    const int64_t j0 = int64_t(ht) * kHops;      // first output hop block

    // this wavefront's frames: samples and band data are requested first
    const float *p = region<float>(a.ws, L.p) + int64_t(row) * L.len;
    const int band_l = lane < kBands ? lane : kBands - 1;
    float smp[kFPW][8], bk_v[kFPW], gbk_v[kFPW], keep[kFPW];
#pragma unroll
    for (int f = 0; f < kFPW; ++f) {
        const int64_t frame = j0 - 1 + wave + kW * f;
        const int64_t fc = frame < 0 ? 0 : (frame >= L.frames ? L.frames - 1 : frame);
        load_frame(p, fc * kHop, L.len, lane, smp[f]);
        const int64_t fo = fc * kBands;
        bk_v[f] = region<float>(a.ws, L.bark)[int64_t(row) * L.frames * kBands + fo + band_l];
        gbk_v[f] = region<float>(a.bw, L.gbark)[int64_t(row) * L.frames * kBands + fo + band_l];
        keep[f] = region<float>(a.ws, L.keep)[int64_t(item) * L.frames + fc];
    }

    // adjoint of the band power ratio and its clamp, then of the mean band
    // powers: wavefront w < kGradSlices sums the band partials of tiles w,
    // w + kGradSlices, ... and every wavefront adds the slices in order
    const double *grp = region<double>(a.bw, L.grpart) + int64_t(item) * L.ntile * kBands;
    if (lane < kBands && !L.totals && wave < kGradSlices) {
        gpart[wave][lane] = tile_partial(grp, L.ntile, wave, kGradSlices, lane, kBands);
    }
    for (int k = threadIdx.x; k < kNfft; k += kWave * kW) {
        if (k < kPassTwiddles) lds_pass[k] = StagedTwiddles<real>::pass(t)[k];
        if (k < kHalf) {
            lds_tw512[k] = StagedTwiddles<real>::fold(t)[k];
            lds_bin_band[k] = t.bin_band[k];
        }
        lds_win[k] = t.window[k];
    }
    __syncthreads();
    double gm = 0.0, th100 = 0.0, corr = 0.0;
    if (lane < kBands) {
        double g = 0.0;
        if (L.totals) {
            g = region<double>(a.bw, L.gradtot)[int64_t(item) * kBands + lane];
        } else {
            for (int w = 0; w < kGradSlices; ++w) g += gpart[w][lane];
        }
        const double ratio = band_array(a, kRatio)[item * kBands + lane];
        const double mref = band_array(a, kMref)[item * kBands + lane];
        const double gr = (ratio >= 0.01 && ratio <= 100.0) ? g : 0.0;
        const double inv = 1.0 / (mref + 1000.0);
        gm = (is_ref ? -gr * ratio * inv : gr * inv) / static_cast<double>(L.frames);
        th100 = 100.0 * t.threshs[lane];
        corr = t.corr[lane];
    }

    const double scale = region<double>(a.ws, L.rowconst)[int64_t(row) * 4 + 2];
    const real s = static_cast<real>(scale) * real(0.5);  // the transform returns 2 X
    cplx<real> *buf = fftbuf[wave];
    // twiddles read per pass from LDS (fewer live registers: five wavefronts
    // per SIMD)
    const LdsTwiddles<real> tw{lds_pass, lds_tw512, lane};
    float win[8];
    int bin_band[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) {
        win[2 * r] = lds_win[2 * (lane + 64 * r)];
        win[2 * r + 1] = lds_win[2 * (lane + 64 * r) + 1];
        bin_band[r] = lds_bin_band[lane + 64 * r];
    }
#pragma unroll
    for (int f = 0; f < kFPW; ++f) {
        const int local = wave + kW * f;
        const int64_t frame = j0 - 1 + local;
        if (frame < 0 || frame >= L.frames) {
            for (int k = lane; k < kNfft; k += kWave) contrib[local][k] = 0.0f;
            continue;
        }
        if (lane < kBands) {
            double g = gbk_v[f];
            if (keep[f] != 0.0f && static_cast<double>(bk_v[f]) > th100) g += gm;
            gband[wave][lane] = static_cast<float>(g * corr);
        }
        wave_lds_fence();
        auto u = [&](int k) -> real {
            const int idx = 2 * (k >> 7) + (k & 1);
            return static_cast<real>(smp[f][idx]) * static_cast<real>(win[idx]);
        };
        cplx<real> x[4];
        frame_spectrum<real, true>(u, x, buf, tw, lane);
        cplx<real> v[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int band = bin_band[r];
            const real gpw = band >= 0 ? static_cast<real>(gband[wave][band]) * s : real(0);
            v[r] = {gpw * x[r].re, gpw * x[r].im};
        }
        real ev[4], od[4];
        frame_adjoint<real>(v, ev, od, buf, tw, lane);
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int n = lane + 64 * r;
            contrib[local][2 * n] = static_cast<float>(ev[r] * static_cast<real>(win[2 * r]));
            contrib[local][2 * n + 1] = static_cast<float>(od[r] * static_cast<real>(win[2 * r + 1]));
        }
        wave_lds_fence();  // gband and the frame buffer are reused by the next frame
    }
    __syncthreads();

    // overlap-add: hop block j0 + q receives frames j0 + q - 1 (second half) and
    // j0 + q; four consecutive samples per thread (16-byte LDS reads, global
    // loads and stores), element by element at the end of the row.  A hop
    // block is one wavefront's pass (wavefront q mod kW, lane l its samples
    // 4 l .. 4 l + 3), whose lane sum is the block's partial of S.
    float *gp_out = region<float>(a.bw, L.gp) + int64_t(i) * L.len;
    double *s_part = region<double>(a.bw, L.spart) + int64_t(i) * L.nhop;
    for (int g4 = threadIdx.x; g4 < kHops * kHop / 4; g4 += blockDim.x) {
        const int k = 4 * g4;
        const int q = k / kHop, m = k % kHop;
        const int64_t hop = j0 + q;  // the same for the whole wavefront
        if (hop >= L.nhop) break;
        const int64_t n = hop * kHop + m;
        double acc = 0.0;
        float lo[4], hi[4], pv[4], out[4];
        __builtin_memcpy(hi, &contrib[q][kHop + m], sizeof(hi));
        __builtin_memcpy(lo, &contrib[q + 1][m], sizeof(lo));
        if (n + 4 <= L.len) {
            __builtin_memcpy(pv, p + n, sizeof(pv));
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const double g = static_cast<double>(hi[e]) + static_cast<double>(lo[e]);
                out[e] = static_cast<float>(g);
                acc = fma(g, static_cast<double>(pv[e]), acc);
            }
            __builtin_memcpy(gp_out + n, out, sizeof(out));
        } else {
            for (int e = 0; e < 4 && n + e < L.len; ++e) {
                const double g = static_cast<double>(hi[e]) + static_cast<double>(lo[e]);
                gp_out[n + e] = static_cast<float>(g);
                acc = fma(g, static_cast<double>(p[n + e]), acc);
            }
        }
        acc = wave_sum(acc);
        if (lane == 0) s_part[hop] = acc;
    }
}

// ---------------------------------------------------------------------------
// stand-alone perceptual chain: silent frames + band partials from given
// spectra, and the mean band power scatter of the backward
// ---------------------------------------------------------------------------

template <int kBPL>
__global__ void __launch_bounds__(kWave) chain_partials_kernel(PipeArgs a) {
    const ModelTable &t = *a.tab;
    const PipeLayout &L = a.L;
    const int nb = L.nb;
    const int item = blockIdx.x / L.ntile;
    const int tile = blockIdx.x - item * L.ntile;
    const int t0 = tile * kTile;
    const int lane = threadIdx.x;
    bool live[kBPL];
    double th100[kBPL], pr[kBPL], pd[kBPL];
#pragma unroll
    for (int k = 0; k < kBPL; ++k) {
        live[k] = lane + kWave * k < nb;
        th100[k] = live[k] ? 100.0 * t.threshs[lane + kWave * k] : 0.0;
        pr[k] = pd[k] = 0.0;
    }
    const float *bref = a.bark_ref + int64_t(item) * L.frames * nb;
    const float *bdeg = a.bark_deg + int64_t(item) * L.frames * nb;
    for (int local = 0; local < kTile; ++local) {
        const int64_t frame = t0 + local;
        if (frame >= L.frames) break;
        double rv[kBPL], dv[kBPL];
        double aud = 0.0;
#pragma unroll
        for (int k = 0; k < kBPL; ++k) {
            const int64_t o = frame * nb + lane + kWave * k;
            rv[k] = live[k] ? static_cast<double>(bref[o]) : 0.0;
            dv[k] = live[k] ? static_cast<double>(bdeg[o]) : 0.0;
            const double x = live[k] && rv[k] > th100[k] ? rv[k] : 0.0;
            aud = k == 0 ? x : aud + x;
        }
        const double total = wave_sum(aud);
        const bool keep = total >= 1e7;
        if (lane == 0) region<float>(a.ws, L.keep)[int64_t(item) * L.frames + frame] = keep ? 1.0f : 0.0f;
#pragma unroll
        for (int k = 0; k < kBPL; ++k) {
            if (keep && rv[k] > th100[k]) pr[k] += rv[k];
            if (keep && dv[k] > th100[k]) pd[k] += dv[k];
        }
    }
#pragma unroll
    for (int k = 0; k < kBPL; ++k) {
        if (!live[k]) continue;
        const int64_t o = (int64_t(item) * L.ntile + tile) * nb + lane + kWave * k;
        region<double>(a.ws, L.bandref)[o] = pr[k];
        region<double>(a.ws, L.banddeg)[o] = pd[k];
    }
}

template <int kBPL>
__global__ void __launch_bounds__(kWave) chain_meanpow_kernel(PipeArgs a) {
    const ModelTable &t = *a.tab;
    const PipeLayout &L = a.L;
    const int nb = L.nb;
    const int item = blockIdx.x / L.ntile;
    const int tile = blockIdx.x - item * L.ntile;
    const int t0 = tile * kTile;
    const int lane = threadIdx.x;
    const double *gp = region<double>(a.bw, L.grpart) + int64_t(item) * L.ntile * nb;
    const float *keep = region<float>(a.ws, L.keep) + int64_t(item) * L.frames;
    const double frames_f = static_cast<double>(L.frames);
#pragma unroll
    for (int k = 0; k < kBPL; ++k) {
        const int band = lane + kWave * k;
        if (band >= nb) continue;
        // the summation order of stft_bwd_kernel: the partial of each of its
        // wavefronts (tiles w, w + kBwdFrames, ...), then those in order; the
        // loads of all of them in flight together
        const double *ptr[kBwdFrames];
        int cnt[kBwdFrames];
#pragma unroll
        for (int w = 0; w < kBwdFrames; ++w) {
            ptr[w] = gp + int64_t(w) * nb + band;
            cnt[w] = L.ntile > w ? static_cast<int>((L.ntile - 1 - w) / kBwdFrames) + 1 : 0;
        }
        double parts[kBwdFrames];
        strided_sums(ptr, cnt, int64_t(kBwdFrames) * nb, parts);
        double g = 0.0;
#pragma unroll
        for (int w = 0; w < kBwdFrames; ++w) g += parts[w];
        const double ratio = band_array(a, kRatio)[item * nb + band];
        const double mref = band_array(a, kMref)[item * nb + band];
        const double gr = (ratio >= 0.01 && ratio <= 100.0) ? g : 0.0;
        const double inv = 1.0 / (mref + 1000.0);
        const double gm_ref = -gr * ratio * inv / frames_f;
        const double gm_deg = gr * inv / frames_f;
        const double th100 = 100.0 * t.threshs[band];
        for (int local = 0; local < kTile; ++local) {
            const int64_t frame = t0 + local;
            if (frame >= L.frames) break;
            if (keep[frame] == 0.0f) continue;
            const int64_t o = (int64_t(item) * L.frames + frame) * nb + band;
            if (static_cast<double>(a.bark_ref[o]) > th100) {
                a.gbark_ref[o] = static_cast<float>(static_cast<double>(a.gbark_ref[o]) + gm_ref);
            }
            if (static_cast<double>(a.bark_deg[o]) > th100) {
                a.gbark_deg[o] = static_cast<float>(static_cast<double>(a.gbark_deg[o]) + gm_deg);
            }
        }
    }
}

// ---------------------------------------------------------------------------
// stand-alone STFT / Bark (the TritonStftBark operator): independent rows,
// no level scale, frames laid over n_padded samples (zero beyond len)
// ---------------------------------------------------------------------------

struct StftArgs {
    const ModelTable *tab;
    const float *x;       // [rows, len]
    float *bark;          // [rows, frames, 49]
    const float *gbark;   // [rows, frames, 49]
    float *gx;            // [rows, len]
    int64_t rows, len, frames, nhoptile, ftiles;
};

constexpr int kPlainWaves = 8;

template <typename real>
__global__ void __launch_bounds__(kWave *kPlainWaves) stft_plain_fwd_kernel(StftArgs a) {
    __shared__ cplx<real> fftbuf[kPlainWaves][kHalf];
    const ModelTable &t = *a.tab;
    const int64_t row = blockIdx.x / a.ftiles;
    const int64_t ft = blockIdx.x - row * a.ftiles;
    const int wave = wave_index();
    const int lane = threadIdx.x % kWave;
    const int64_t frame = ft * kPlainWaves + wave;
    if (frame >= a.frames) return;
    const float *x = a.x + row * a.len;
    const int64_t start = frame * kHop;
    auto u = [&](int k) -> real {
        const int64_t n = start + k;
        return static_cast<real>(load_or_zero(x, n, a.len)) * static_cast<real>(t.window[k]);
    };
    cplx<real> *buf = fftbuf[wave];
    cplx<real> spec[4];
    Twiddles<real> tw;
    tw.load(t.tw256, t.tw512, lane);
    frame_spectrum<real>(u, spec, buf, tw, lane);
    real *power = reinterpret_cast<real *>(buf);
#pragma unroll
    for (int r = 0; r < 4; ++r) {
        const int f = lane + 64 * r;
        power[f] = f == 0 ? real(0) : spec[r].re * spec[r].re + spec[r].im * spec[r].im;
    }
    wave_lds_fence();
    if (lane < kBands) {
        double acc = 0.0;
        for (int f = t.band_start[lane]; f < t.band_end[lane]; ++f) acc += static_cast<double>(power[f]);
        a.bark[(row * a.frames + frame) * kBands + lane] = static_cast<float>(acc * t.corr[lane]);
    }
}

template <typename real>
__global__ void __launch_bounds__(kWave *kBwdFrames) stft_plain_bwd_kernel(StftArgs a) {
    __shared__ cplx<real> fftbuf[kBwdFrames][kHalf];
    __shared__ float contrib[kBwdFrames][kNfft];
    __shared__ float gband[kBwdFrames][kBands];
    const ModelTable &t = *a.tab;
    const int64_t row = blockIdx.x / a.nhoptile;
    const int64_t ht = blockIdx.x - row * a.nhoptile;
    const int wave = wave_index();
    const int lane = threadIdx.x % kWave;
    const int64_t j0 = ht * kBwdHops;
    const int64_t frame = j0 - 1 + wave;
    const float *x = a.x + row * a.len;
    if (frame >= 0 && frame < a.frames) {
        if (lane < kBands) {
            gband[wave][lane] = static_cast<float>(
                static_cast<double>(a.gbark[(row * a.frames + frame) * kBands + lane]) * t.corr[lane]);
        }
        wave_lds_fence();
        const int64_t start = frame * kHop;
        auto u = [&](int k) -> real {
            const int64_t n = start + k;
            return static_cast<real>(load_or_zero(x, n, a.len)) * static_cast<real>(t.window[k]);
        };
        cplx<real> spec[4], v[4];
        Twiddles<real> tw;
        tw.load(t.tw256, t.tw512, lane);
        frame_spectrum<real>(u, spec, fftbuf[wave], tw, lane);
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int band = t.bin_band[lane + 64 * r];
            const real g = band >= 0 ? static_cast<real>(gband[wave][band]) : real(0);
            v[r] = {g * spec[r].re, g * spec[r].im};
        }
        real ev[4], od[4];
        frame_adjoint<real>(v, ev, od, fftbuf[wave], tw, lane);
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int n = lane + 64 * r;
            contrib[wave][2 * n] = static_cast<float>(ev[r] * static_cast<real>(t.window[2 * n]));
            contrib[wave][2 * n + 1] = static_cast<float>(od[r] * static_cast<real>(t.window[2 * n + 1]));
        }
    } else {
        for (int k = lane; k < kNfft; k += kWave) contrib[wave][k] = 0.0f;
    }
    __syncthreads();
    float *gx = a.gx + row * a.len;
    for (int k = threadIdx.x; k < kBwdHops * kHop; k += blockDim.x) {
        const int q = k / kHop, m = k % kHop;
        const int64_t n = (j0 + q) * kHop + m;
        if (n >= a.len) continue;
        gx[n] = static_cast<float>(static_cast<double>(contrib[q][kHop + m]) +
                                   static_cast<double>(contrib[q + 1][m]));
    }
}

// ---------------------------------------------------------------------------
// host entry points
// ---------------------------------------------------------------------------

// FFT arithmetic of the stand-alone STFT operator: float64.
#ifndef PESQ_STFT_REAL
#define PESQ_STFT_REAL double
#endif
using StftReal = PESQ_STFT_REAL;
// FFT arithmetic of the fused forward STFT of small grids (latency bound) and
// of large grids (throughput bound): float32 passes, twiddles and bins, with
// the band sums in float64.  The kernels are bound by LDS traffic and issue,
// and float32 halves the LDS bytes of every pass and the registers (five
// wavefronts per SIMD at large grids instead of four): 98 instead of 142 us at
// BASELINE c5, 11.2 instead of 14.4 us at c2.  The distances then differ from
// float64 by up to 2.5e-6 at c5 and 4e-7 at c2 (5e-7 and 7e-8 with float64
// passes), within the 1e-5 bound.
#ifndef PESQ_STFT_FUSED_REAL
#define PESQ_STFT_FUSED_REAL float
#endif
#ifndef PESQ_STFT_LEAN_REAL
#define PESQ_STFT_LEAN_REAL float
#endif
using StftFusedReal = PESQ_STFT_FUSED_REAL;
using StftLeanReal = PESQ_STFT_LEAN_REAL;
// The backward's FFTs (spectrum recomputed, adjoint) run in float32: fewer
// registers (five wavefronts per SIMD instead of four; 20.3 instead of 22.9 us
// at BASELINE c2) for a gradient error of about 2e-6 of its peak instead of
// 5e-7.
using StftBwdReal = float;

// Chain launches: up to about two workgroups per CU of the 256 CU MI355X
// (kWideTiles chain tiles) the kernels are latency bound and run one frame
// (backward) or two (forward) per wavefront; larger grids run four frames per
// wavefront (measured best at BASELINE c2 and c5 respectively).  The results
// are the same either way.

// The kernel variants the pipeline launches for one shape.  Every launch
// below and pesq_pipeline_kernels read this one plan, so the variants a test
// asks about are the ones that run.
struct PipePlan {
    ScanPlan fwd_scan, bwd_scan;
    bool stft_lean;      // stft_fwd_kernel<.., true>: grids above kWideTiles
    int chain_fwd_waves, chain_bwd_waves;
    int chain_bpl;       // bands per lane: 1 up to 64 bands, 2 up to 128
};

static PipePlan pipe_plan(const PipeLayout &L) {
    PipePlan P{};
    P.fwd_scan = scan_plan(L.rows, L.nblk);
    P.bwd_scan = scan_plan(L.nrg, L.nblk);
    const int64_t grid = L.batch * L.ntile;
    const bool wide = grid > kWideTiles;
    P.stft_lean = wide;
    // Up to 64 bands a lane holds one band; 65 .. 128 bands take two per lane
    // (band lane + 64), with 4 wavefronts per workgroup for the larger
    // register footprint.
    P.chain_bpl = L.nb > kWave ? 2 : 1;
    P.chain_fwd_waves = P.chain_bpl == 2 || wide ? 4 : 8;
    P.chain_bwd_waves = P.chain_bpl == 2 || wide ? 4 : 16;
    return P;
}

static void launch_chain_fwd(const PipeArgs &a, unsigned grid, hipStream_t stream) {
    const PipePlan P = pipe_plan(a.L);
    if (P.chain_bpl == 2) {
        hipLaunchKernelGGL((chain_fwd_kernel<4, 2>), dim3(grid), dim3(kWave * 4), 0, stream, a);
    } else if (P.chain_fwd_waves == 8) {
        hipLaunchKernelGGL((chain_fwd_kernel<8, 1>), dim3(grid), dim3(kWave * 8), 0, stream, a);
    } else {
        hipLaunchKernelGGL((chain_fwd_kernel<4, 1>), dim3(grid), dim3(kWave * 4), 0, stream, a);
    }
}

static void launch_chain_bwd(const PipeArgs &a, unsigned grid, hipStream_t stream) {
    const PipePlan P = pipe_plan(a.L);
    if (P.chain_bpl == 2) {
        hipLaunchKernelGGL((chain_bwd_kernel<4, 2>), dim3(grid), dim3(kWave * 4), 0, stream, a);
    } else if (P.chain_bwd_waves == 16) {
        hipLaunchKernelGGL((chain_bwd_kernel<16, 1>), dim3(grid), dim3(kWave * 16), 0, stream, a);
    } else {
        hipLaunchKernelGGL((chain_bwd_kernel<4, 1>), dim3(grid), dim3(kWave * 4), 0, stream, a);
    }
}

#ifndef PESQ_SPLIT_AGGREGATE
#define PESQ_SPLIT_AGGREGATE 1
#endif
// the scans' aggregate pass of lane-state grids by kSplitWaves wavefronts per block
constexpr bool kSplitAggregate = PESQ_SPLIT_AGGREGATE != 0;

// Names of the kernels of one scan pass, in launch order (host_power: the
// backward scan is its output launch alone).
static void scan_kernel_names(const ScanPlan &S, const char *mode, std::string &out,
                              bool host_power = false) {
    const char *lanes = S.lane_states ? "true" : "false";
    const int prefix = kPipeWindow && S.lane_states
                           ? kWindowStarts
                           : (S.fused_prefix ? kFusedSums : kStoredStarts);
    const std::string output = std::string("iir_output_kernel<5, 1, ") + mode + ", " + lanes +
                               ", " + std::to_string(prefix) + ", ";
    if (host_power) {
        // no aggregate launch: the level alignment filter's ran in the forward's
        // chain kernel, the pre-emphasis filter warms up in the output pass
        out += kSplitOutput && prefix == kWindowStarts
                   ? std::string("iir_output_split_kernel<5, 1, ") + mode + ", true>;"
                   : output + "true>;";
        return;
    } else if (kSplitAggregate && S.lane_states) {
        out += "iir_aggregate_split_kernel<5, 1, " + std::to_string(kSplitWaves) + ", " + mode +
               ">;";
    } else {
        out += std::string("iir_aggregate_kernel<5, 1, ") + mode + ", " + lanes + ", 0, 6>;";
    }
    if (prefix == kStoredStarts) out += "iir_prefix_kernel<6>;";
    out += output + "false>;";
}

static int check_sizes(int64_t batch, int64_t len, const PipeLayout &L) {
    PESQ_CHECK_ARG(batch >= 0, "batch must not be negative, got %lld", (long long)batch);
    PESQ_CHECK_ARG(len >= 15, "the edge ramp needs at least 15 samples, got %lld", (long long)len);
    PESQ_CHECK_ARG(L.frames >= kWin,
                   "The PESQ chain needs at least 20 frames for the overlapping sums, got %lld",
                   (long long)L.frames);
    PESQ_CHECK_ARG(2 * batch * L.nblk < (int64_t(1) << 31) && 2 * batch * L.ntile < (int64_t(1) << 31),
                   "problem too large for one launch");
    return PESQ_OK;
}

}  // namespace pesq

using namespace pesq;

extern "C" int pesq_pipeline_forward_workspace(int64_t batch, int64_t len, int grad_mask,
                                               size_t *bytes) {
    PipeLayout L;
    L.build(batch, len, grad_mask);
    if (int st = check_sizes(batch, len, L)) return st;
    *bytes = L.fwd_bytes;
    return PESQ_OK;
}

extern "C" int pesq_pipeline_backward_workspace(int64_t batch, int64_t len, int grad_mask,
                                                size_t *bytes) {
    PipeLayout L;
    L.build(batch, len, grad_mask);
    if (int st = check_sizes(batch, len, L)) return st;
    *bytes = L.bwd_bytes;
    return PESQ_OK;
}

extern "C" int pesq_pipeline_region(int64_t batch, int64_t len, int grad_mask, const char *name,
                                    size_t *offset, size_t *bytes) {
    PipeLayout L;
    L.build(batch, len, grad_mask);
    PESQ_CHECK_ARG(name != nullptr && L.region(name, offset, bytes), "unknown region %s",
                   name ? name : "(null)");
    return PESQ_OK;
}

extern "C" int pesq_pipeline_kernels(int64_t batch, int64_t len, int grad_mask, int backward,
                                     char *names, size_t capacity, size_t *needed) {
    PipeLayout L;
    L.build(batch, len, grad_mask);
    if (int st = check_sizes(batch, len, L)) return st;
    PESQ_CHECK_ARG((grad_mask & ~3) == 0, "invalid grad_mask %d", grad_mask);
    PESQ_CHECK_ARG(!backward || grad_mask != 0, "backward needs a non-empty grad_mask");
    const PipePlan P = pipe_plan(L);
    const bool lean_double = std::is_same<StftLeanReal, double>::value;
    const bool fused_double = std::is_same<StftFusedReal, double>::value;
    const char *real = (P.stft_lean ? lean_double : fused_double) ? "double" : "float";
    const char *bwd_real = std::is_same<StftBwdReal, double>::value ? "double" : "float";
    std::string out;
    if (!backward) {
        scan_kernel_names(P.fwd_scan, "PipeFwdMode", out);
        out += std::string("stft_fwd_kernel<") + real + ", " + (P.stft_lean ? "true" : "false") +
               ", " + std::to_string(kStftWaves) + ">;";
        if (L.totals) out += "band_totals_kernel<" + std::to_string(kChainSlices) + ", 2>;";
        out += "chain_fwd_kernel<" + std::to_string(P.chain_fwd_waves) + ", " +
               std::to_string(P.chain_bpl) + ">;";
        out += "chain_final_kernel;";
    } else {
        out += "chain_bwd_kernel<" + std::to_string(P.chain_bwd_waves) + ", " +
               std::to_string(P.chain_bpl) + ">;";
        if (L.totals) out += "band_totals_kernel<" + std::to_string(kGradSlices) + ", 1>;";
        out += std::string("stft_bwd_kernel<") + bwd_real + ", " + std::to_string(L.bwd_fpw) +
               ", " + std::to_string(L.bwd_waves) + ">;";
        scan_kernel_names(P.bwd_scan, "PipeBwdMode", out, L.host_power);
    }
    out.pop_back();  // the last ';'
    if (needed != nullptr) *needed = out.size() + 1;
    if (names != nullptr && capacity > 0) {
        const size_t n = std::min(out.size(), capacity - 1);
        std::memcpy(names, out.data(), n);
        names[n] = '\0';
    }
    return PESQ_OK;
}

extern "C" int pesq_pipeline_forward_stages(const float *ref, const float *deg, int64_t batch,
                                            int64_t len, const void *model_table, double factor,
                                            int grad_mask, float *d_symm, float *d_asymm,
                                            float *mos, float *loss, void *fwd_workspace,
                                            unsigned stages, hipStream_t stream) {
    PipeArgs a{};
    a.L.build(batch, len, grad_mask);
    if (int st = check_sizes(batch, len, a.L)) return st;
    PESQ_CHECK_ARG((grad_mask & ~3) == 0, "invalid grad_mask %d", grad_mask);
    if (batch == 0) return PESQ_OK;  // an empty batch has nothing to score
    PESQ_CHECK_ARG(ref && deg && model_table && fwd_workspace && d_symm && d_asymm && mos && loss,
                   "null pointer argument");
    a.tab = static_cast<const ModelTable *>(model_table);
    a.ref = ref;
    a.deg = deg;
    a.ws = static_cast<unsigned char *>(fwd_workspace);
    a.factor = factor;
    a.d_symm = d_symm;
    a.d_asymm = d_asymm;
    a.mos = mos;
    a.loss = loss;
    const PipeLayout &L = a.L;
    const IirTable *iir = &a.tab->iir;
    a.bark_ref = region<float>(a.ws, L.bark);
    a.bark_deg = a.bark_ref + batch * L.frames * kBands;

    PipeFwdMode m{};
    m.ref = ref;
    m.deg = deg;
    m.p = region<float>(a.ws, L.p);
    m.f = grad_mask ? region<float>(a.ws, L.f) : nullptr;
    m.energy = region<double>(a.ws, L.energy);
    m.len = len;
    m.batch = static_cast<int>(batch);
    m.nblk = static_cast<int>(L.nblk);
    m.row0 = static_cast<int>(L.row0);
    m.nrg = static_cast<int>(L.nrg);
    double *aggr = region<double>(a.ws, L.aggr);

    if (stages & 3u) {
        if (int st = launch_scan<kPowerSections, kPreSections>(m, iir, aggr, L.rows, len,
                                                               stages & 1u, stages & 2u, stream,
                                                               kSplitAggregate, false,
                                                               kPipeWindow)) {
            return st;
        }
    }
    if (stages & 4u) {
        unsigned grid = static_cast<unsigned>(batch * L.ntile);
        // and the backward's level alignment aggregate blocks, a wavefront each
        if (L.host_power) grid += static_cast<unsigned>(cdiv(L.nrg * L.nblk, kStftWaves));
        if (!pipe_plan(L).stft_lean) {
            hipLaunchKernelGGL((stft_fwd_kernel<StftFusedReal, false>), dim3(grid),
                               dim3(kWave * kStftWaves), 0, stream, a);
        } else {
            hipLaunchKernelGGL((stft_fwd_kernel<StftLeanReal, true>), dim3(grid),
                               dim3(kWave * kStftWaves), 0, stream, a);
        }
        PESQ_CHECK_LAUNCH("pipeline stft");
    }
    if (stages & 8u) {
        if (L.totals) {
            hipLaunchKernelGGL((band_totals_kernel<kChainSlices, 2>),
                               dim3(static_cast<unsigned>(batch)), dim3(kWave * kChainSlices), 0,
                               stream, a);
            PESQ_CHECK_LAUNCH("pipeline band totals");
        }
        launch_chain_fwd(a, static_cast<unsigned>(batch * L.ntile), stream);
        PESQ_CHECK_LAUNCH("pipeline chain");
    }
    if (stages & 16u) {
        hipLaunchKernelGGL(chain_final_kernel, dim3(static_cast<unsigned>(batch)),
                           dim3(final_threads(L.nwin)), 0, stream, a);
        PESQ_CHECK_LAUNCH("pipeline chain final");
    }
    return PESQ_OK;
}

extern "C" int pesq_pipeline_forward(const float *ref, const float *deg, int64_t batch,
                                     int64_t len, const void *model_table, double factor,
                                     int grad_mask, float *d_symm, float *d_asymm, float *mos,
                                     float *loss, void *fwd_workspace, hipStream_t stream) {
    return pesq_pipeline_forward_stages(ref, deg, batch, len, model_table, factor, grad_mask,
                                        d_symm, d_asymm, mos, loss, fwd_workspace, 0x1Fu, stream);
}

extern "C" int pesq_pipeline_backward_stages(const float *g_symm, const float *g_asymm,
                                             const float *g_mos, const float *g_loss,
                                             int64_t batch, int64_t len, const void *model_table,
                                             double factor, int grad_mask, float *g_ref,
                                             float *g_deg, const void *fwd_workspace,
                                             void *bwd_workspace, unsigned stages,
                                             hipStream_t stream) {
    PipeArgs a{};
    a.L.build(batch, len, grad_mask);
    if (int st = check_sizes(batch, len, a.L)) return st;
    PESQ_CHECK_ARG(grad_mask >= 1 && grad_mask <= 3, "backward needs a non-empty grad_mask");
    if (batch == 0) return PESQ_OK;
    PESQ_CHECK_ARG(!(grad_mask & PESQ_GRAD_REF) || g_ref, "g_ref is required by grad_mask");
    PESQ_CHECK_ARG(!(grad_mask & PESQ_GRAD_DEG) || g_deg, "g_deg is required by grad_mask");
    PESQ_CHECK_ARG(model_table && fwd_workspace && bwd_workspace, "null pointer argument");
    a.tab = static_cast<const ModelTable *>(model_table);
    a.ws = static_cast<unsigned char *>(const_cast<void *>(fwd_workspace));
    a.bw = static_cast<unsigned char *>(bwd_workspace);
    a.factor = factor;
    a.g_symm = g_symm;
    a.g_asymm = g_asymm;
    a.g_mos = g_mos;
    a.g_loss = g_loss;
    const PipeLayout &L = a.L;
    const IirTable *iir = &a.tab->iir;
    a.bark_ref = region<float>(a.ws, L.bark);
    a.bark_deg = a.bark_ref + batch * L.frames * kBands;
    a.gbark_ref = region<float>(a.bw, L.gbark);
    a.gbark_deg = a.gbark_ref + batch * L.frames * kBands;

    if (stages & 1u) {
        launch_chain_bwd(a, static_cast<unsigned>(batch * L.ntile), stream);
        PESQ_CHECK_LAUNCH("pipeline chain backward");
    }
    if (stages & 2u) {
        if (L.totals) {
            hipLaunchKernelGGL((band_totals_kernel<kGradSlices, 1>),
                               dim3(static_cast<unsigned>(batch)), dim3(kWave * kGradSlices), 0,
                               stream, a);
            PESQ_CHECK_LAUNCH("pipeline gradient totals");
        }
        const dim3 grid(static_cast<unsigned>(L.nrg * L.nhoptile));
        if (L.bwd_fpw == 2) {
            hipLaunchKernelGGL((stft_bwd_kernel<StftBwdReal, 2, kBwdWaves>), grid,
                               dim3(kWave * kBwdWaves), 0, stream, a);
        } else {
            hipLaunchKernelGGL((stft_bwd_kernel<StftBwdReal, 1, kBwdWavesSmall>), grid,
                               dim3(kWave * kBwdWavesSmall), 0, stream, a);
        }
        PESQ_CHECK_LAUNCH("pipeline stft backward");
    }

    PipeBwdMode m{};
    m.f = region<float>(a.ws, L.f);
    m.gp = region<float>(a.bw, L.gp);
    m.rowconst = region<double>(a.ws, L.rowconst);
    m.spart = region<double>(a.bw, L.spart);
    m.g_ref = g_ref;
    m.g_deg = g_deg;
    m.len = len;
    m.batch = static_cast<int>(batch);
    m.row0 = static_cast<int>(L.row0);
    m.nhop = static_cast<int>(L.nhop);
    if (L.host_power) {
        // the level alignment filter's aggregates came from the forward's
        // chain kernel (sections 0..4); the output pass warms the
        // pre-emphasis filter (section 5) up itself and runs both filters
        double *aggr = region<double>(a.ws, L.aggr_b);
        if (stages & 8u) {
            return launch_scan<kPowerSections, kPreSections>(m, iir, aggr, L.nrg, len, false,
                                                             true, stream, false, true,
                                                             kPipeWindow);
        }
        return PESQ_OK;
    }
    double *aggr = region<double>(a.bw, L.aggr_b);
    if (stages & 12u) {
        return launch_scan<kPowerSections, kPreSections>(m, iir, aggr, L.nrg, len, stages & 4u,
                                                         stages & 8u, stream, kSplitAggregate,
                                                         false, kPipeWindow);
    }
    return PESQ_OK;
}

extern "C" int pesq_pipeline_backward(const float *g_symm, const float *g_asymm,
                                      const float *g_mos, const float *g_loss, int64_t batch,
                                      int64_t len, const void *model_table, double factor,
                                      int grad_mask, float *g_ref, float *g_deg,
                                      const void *fwd_workspace, void *bwd_workspace,
                                      hipStream_t stream) {
    return pesq_pipeline_backward_stages(g_symm, g_asymm, g_mos, g_loss, batch, len, model_table,
                                         factor, grad_mask, g_ref, g_deg, fwd_workspace,
                                         bwd_workspace, 0xFu, stream);
}

// ---------------------------------------------------------------------------
// stand-alone chain and STFT entry points
// ---------------------------------------------------------------------------

static int chain_args(PipeArgs &a, int64_t batch, int64_t frames, int nbands,
                      const void *model_table) {
    PESQ_CHECK_ARG(batch >= 0, "batch must not be negative, got %lld", (long long)batch);
    PESQ_CHECK_ARG(nbands >= 1 && nbands <= kMaxChainBands, "the chain takes 1 .. %d bands, got %d",
                   kMaxChainBands, nbands);
    PESQ_CHECK_ARG(frames >= kWin,
                   "The PESQ chain needs at least 20 frames for the overlapping sums, got %lld",
                   (long long)frames);
    PESQ_CHECK_ARG(batch * cdiv(frames, kTile) < (int64_t(1) << 31), "problem too large for one launch");
    PESQ_CHECK_ARG(model_table != nullptr, "null model table");
    a.L.build_chain(batch, frames, nbands);
    a.tab = static_cast<const ModelTable *>(model_table);
    return PESQ_OK;
}

extern "C" int pesq_chain_forward_workspace(int64_t batch, int64_t frames, int nbands,
                                            size_t *bytes) {
    PipeArgs a{};
    if (int st = chain_args(a, batch, frames, nbands, reinterpret_cast<const void *>(1))) return st;
    *bytes = a.L.fwd_bytes;
    return PESQ_OK;
}

extern "C" int pesq_chain_backward_workspace(int64_t batch, int64_t frames, int nbands,
                                             size_t *bytes) {
    PipeArgs a{};
    if (int st = chain_args(a, batch, frames, nbands, reinterpret_cast<const void *>(1))) return st;
    *bytes = a.L.bwd_bytes;
    return PESQ_OK;
}

extern "C" int pesq_chain_forward(const float *ref_bark, const float *deg_bark, int64_t batch,
                                  int64_t frames, int nbands, const void *model_table,
                                  float *d_symm, float *d_asymm, void *fwd_workspace,
                                  hipStream_t stream) {
    PipeArgs a{};
    if (int st = chain_args(a, batch, frames, nbands, model_table)) return st;
    if (batch == 0) return PESQ_OK;  // test_triton_chain.py:799-806: a no-op
    PESQ_CHECK_ARG(ref_bark && deg_bark && d_symm && d_asymm && fwd_workspace, "null pointer argument");
    a.ws = static_cast<unsigned char *>(fwd_workspace);
    a.bark_ref = ref_bark;
    a.bark_deg = deg_bark;
    a.d_symm = d_symm;
    a.d_asymm = d_asymm;
    const unsigned grid = static_cast<unsigned>(batch * a.L.ntile);
    if (a.L.nb > kWave) {
        hipLaunchKernelGGL(chain_partials_kernel<2>, dim3(grid), dim3(kWave), 0, stream, a);
    } else {
        hipLaunchKernelGGL(chain_partials_kernel<1>, dim3(grid), dim3(kWave), 0, stream, a);
    }
    PESQ_CHECK_LAUNCH("chain partials");
    launch_chain_fwd(a, grid, stream);
    PESQ_CHECK_LAUNCH("chain");
    hipLaunchKernelGGL(chain_final_kernel, dim3(static_cast<unsigned>(batch)),
                       dim3(final_threads(a.L.nwin)), 0, stream, a);
    PESQ_CHECK_LAUNCH("chain final");
    return PESQ_OK;
}

extern "C" int pesq_chain_backward(const float *g_symm, const float *g_asymm, const float *ref_bark,
                                   const float *deg_bark, int64_t batch, int64_t frames,
                                   int nbands, const void *model_table, float *g_ref_bark,
                                   float *g_deg_bark, const void *fwd_workspace,
                                   void *bwd_workspace, hipStream_t stream) {
    PipeArgs a{};
    if (int st = chain_args(a, batch, frames, nbands, model_table)) return st;
    if (batch == 0) return PESQ_OK;
    PESQ_CHECK_ARG(ref_bark && deg_bark && g_ref_bark && g_deg_bark && fwd_workspace && bwd_workspace,
                   "null pointer argument");
    a.ws = static_cast<unsigned char *>(const_cast<void *>(fwd_workspace));
    a.bw = static_cast<unsigned char *>(bwd_workspace);
    a.bark_ref = ref_bark;
    a.bark_deg = deg_bark;
    a.gbark_ref = g_ref_bark;
    a.gbark_deg = g_deg_bark;
    a.g_symm = g_symm;
    a.g_asymm = g_asymm;
    const unsigned grid = static_cast<unsigned>(batch * a.L.ntile);
    launch_chain_bwd(a, grid, stream);
    PESQ_CHECK_LAUNCH("chain backward");
    if (a.L.nb > kWave) {
        hipLaunchKernelGGL(chain_meanpow_kernel<2>, dim3(grid), dim3(kWave), 0, stream, a);
    } else {
        hipLaunchKernelGGL(chain_meanpow_kernel<1>, dim3(grid), dim3(kWave), 0, stream, a);
    }
    PESQ_CHECK_LAUNCH("chain mean power backward");
    return PESQ_OK;
}

static int stft_args(StftArgs &a, int64_t rows, int64_t len, int64_t n_padded, const void *table) {
    PESQ_CHECK_ARG(rows >= 0 && len >= 0, "invalid sizes");
    PESQ_CHECK_ARG(n_padded >= len, "n_padded (%lld) is smaller than the signal length (%lld)",
                   (long long)n_padded, (long long)len);
    PESQ_CHECK_ARG(n_padded >= kNfft, "n_padded (%lld) is shorter than one frame (512)",
                   (long long)n_padded);
    PESQ_CHECK_ARG(table != nullptr, "null model table");
    a.tab = static_cast<const ModelTable *>(table);
    a.rows = rows;
    a.len = len;
    a.frames = 1 + (n_padded - kNfft) / kHop;
    a.ftiles = cdiv(a.frames, kPlainWaves);
    a.nhoptile = cdiv(cdiv(len, kHop), kBwdHops);
    PESQ_CHECK_ARG(rows * a.ftiles < (int64_t(1) << 31) && rows * a.nhoptile < (int64_t(1) << 31),
                   "problem too large for one launch");
    return PESQ_OK;
}

extern "C" int pesq_stft_bark_forward(const float *x, int64_t rows, int64_t len, int64_t n_padded,
                                      const void *model_table, float *bark, hipStream_t stream) {
    StftArgs a{};
    if (int st = stft_args(a, rows, len, n_padded, model_table)) return st;
    if (rows == 0) return PESQ_OK;
    PESQ_CHECK_ARG(x && bark, "null pointer argument");
    a.x = x;
    a.bark = bark;
    hipLaunchKernelGGL(stft_plain_fwd_kernel<StftReal>, dim3(static_cast<unsigned>(rows * a.ftiles)),
                       dim3(kWave * kPlainWaves), 0, stream, a);
    PESQ_CHECK_LAUNCH("stft bark forward");
    return PESQ_OK;
}

extern "C" int pesq_stft_bark_backward(const float *g_bark, const float *x, int64_t rows,
                                       int64_t len, int64_t n_padded, const void *model_table,
                                       float *g_x, hipStream_t stream) {
    StftArgs a{};
    if (int st = stft_args(a, rows, len, n_padded, model_table)) return st;
    if (rows == 0 || len == 0) return PESQ_OK;
    PESQ_CHECK_ARG(x && g_bark && g_x, "null pointer argument");
    a.x = x;
    a.gbark = g_bark;
    a.gx = g_x;
    hipLaunchKernelGGL(stft_plain_bwd_kernel<StftReal>, dim3(static_cast<unsigned>(rows * a.nhoptile)),
                       dim3(kWave * kBwdFrames), 0, stream, a);
    PESQ_CHECK_LAUNCH("stft bark backward");
    return PESQ_OK;
}
