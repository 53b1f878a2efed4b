// Framed 512 point real FFT for the STFT / Bark stage, one wavefront per frame.
//
// A 512 point real frame u is folded into the 256 point complex sequence
// z_n = u_{2n} + i u_{2n+1}; Z = FFT256(z) is computed by a radix-4 Stockham
// autosort FFT (4 passes) whose 64 butterflies per pass are the 64 lanes of
// the wavefront, with the sequence held in a wave-private LDS buffer.  The
// half spectrum follows from
//     X_f = (Z_f + conj Z_{256-f}) / 2 - i e^{-2 pi i f / 512} (Z_f - conj Z_{256-f}) / 2.
// The backward pass needs the adjoint g_u_k = sum_f V_f e^{+2 pi i f k / 512}
// of a Hermitian V (V_f = gP_f X_f for f = 1..255, zero at DC and Nyquist),
// obtained from the inverse of the same fold:
//     Z'_f = (V_f + conj V_{256-f}) + i e^{+2 pi i f / 512} (V_f - conj V_{256-f}),
//     z = IFFT256(Z') (unnormalised),  g_u_{2n} = Re z_n,  g_u_{2n+1} = Im z_n.
//
// Rounding.  Floating point contraction is off in every function here and in
// the kernels that use them: each product that meets a sum is either an
// explicit fused multiply-add (fmadd) or rounded on its own, as written.  The
// compiler would otherwise choose which products to fuse per instantiation,
// and the launch variants of one transform (registers or LDS twiddles, one or
// two frames per wavefront) would round differently; written out, every
// variant computes the same bits for a frame.
#pragma once

#include "common.hpp"

namespace pesq {

constexpr int kNfft = 512;
constexpr int kHop = 256;
constexpr int kHalf = 256;
constexpr int kBands = 49;
constexpr int kMaxBandBins = 25;  // widest Bark band of the 16 kHz table (bins)

// The 8 samples of a 512 sample frame that lane `lane` folds into its 4 complex
// inputs: s[2 r + e] = x[start + 2 (lane + 64 r) + e] (zero past len).  A frame
// that ends inside the row (all but the padded last one) loads its pairs
// without bounds checks.
__device__ __forceinline__ void load_frame(const float *x, int64_t start, int64_t len, int lane,
                                           float (&s)[8]) {
    if (start + kNfft <= len) {
        const float *f = x + start + 2 * lane;
#pragma unroll
        for (int r = 0; r < 4; ++r) __builtin_memcpy(&s[2 * r], f + 128 * r, 2 * sizeof(float));
        return;
    }
#pragma unroll
    for (int r = 0; r < 4; ++r) {
#pragma unroll
        for (int e = 0; e < 2; ++e) s[2 * r + e] = load_or_zero(x, start + 2 * (lane + 64 * r) + e, len);
    }
}

template <typename real>
struct cplx {
    real re, im;
};

__device__ __forceinline__ float fmadd(float a, float b, float c) { return __builtin_fmaf(a, b, c); }
__device__ __forceinline__ double fmadd(double a, double b, double c) { return __builtin_fma(a, b, c); }

template <typename real>
__device__ __forceinline__ cplx<real> cmul(cplx<real> a, cplx<real> b) {
#pragma clang fp contract(off)
    return {fmadd(a.re, b.re, -(a.im * b.im)), fmadd(a.re, b.im, a.im * b.re)};
}

// radix-4 DFT of v[0..3]; forward uses e^{-2 pi i / 4} = -i
template <typename real, bool kInverse>
__device__ __forceinline__ void dft4(cplx<real> (&v)[4]) {
#pragma clang fp contract(off)
    const cplx<real> a0 = {v[0].re + v[2].re, v[0].im + v[2].im};
    const cplx<real> a1 = {v[0].re - v[2].re, v[0].im - v[2].im};
    const cplx<real> a2 = {v[1].re + v[3].re, v[1].im + v[3].im};
    const cplx<real> d = {v[1].re - v[3].re, v[1].im - v[3].im};
    // forward: a3 = -i d, inverse: a3 = +i d
    const cplx<real> a3 = kInverse ? cplx<real>{-d.im, d.re} : cplx<real>{d.im, -d.re};
    v[0] = {a0.re + a2.re, a0.im + a2.im};
    v[2] = {a0.re - a2.re, a0.im - a2.im};
    v[1] = {a1.re + a3.re, a1.im + a3.im};
    v[3] = {a1.re - a3.re, a1.im - a3.im};
}

// LDS slot of complex element i of a frame buffer.  The radix-4 passes write
// elements 4 l + r and 16 (l / 4) + l % 4 + 4 r from lane l, which put the 16
// lanes of one LDS cycle on only 4 different bank groups of a 16-byte element;
// xoring bits 4-5 of the index into bits 0-3 (times 5) spreads every pass over
// all 16 groups and keeps the unit stride reads conflict free.
__device__ __forceinline__ int slot(int i) { return i ^ (((i >> 4) & 3) * 5); }

// Power of the band [lo, hi) of every lane from the 256 bins p[0 .. 255] of
// the wave's LDS buffer, through a float64 prefix sum: lane l adds bins
// 4 l .. 4 l + 3 in order, a wave scan turns the lane totals into
// S_k = sum_{g <= k} p_g, and the band is S_{hi-1} - S_{lo-1}.  Its rounding
// is a few units of 2^-53 of the frame's total power, far below the float32
// rounding of the band value.  The prefix sums overwrite the buffer (kHalf
// doubles, which the frame buffer holds for float and double bins alike).
template <typename real>
__device__ __forceinline__ double band_power(real *p, int lane, int lo, int hi) {
#pragma clang fp contract(off)
    real b[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) b[j] = p[4 * lane + j];
    double s[4];
    s[0] = static_cast<double>(b[0]);
#pragma unroll
    for (int j = 1; j < 4; ++j) s[j] = s[j - 1] + static_cast<double>(b[j]);
    const double before = wave_shift_up(wave_inclusive_scan(s[3]));
    wave_lds_fence();
    double *prefix = reinterpret_cast<double *>(p);
#pragma unroll
    for (int j = 0; j < 4; ++j) prefix[4 * lane + j] = before + s[j];
    wave_lds_fence();
    const double upper = hi > 0 ? prefix[hi - 1] : 0.0;
    const double lower = lo > 0 ? prefix[lo - 1] : 0.0;
    wave_lds_fence();
    return upper - lower;
}

// Two-component vector of the twiddle tables staged in LDS for an FFT in
// `real` arithmetic (the tables are stored in the arithmetic's precision).
template <typename real>
struct Vec2;
template <>
struct Vec2<float> {
    using type = float2;
};
template <>
struct Vec2<double> {
    using type = double2;
};

template <typename real>
__device__ __forceinline__ typename Vec2<real>::type to_vec2(double2 w) {
    return {static_cast<real>(w.x), static_cast<real>(w.y)};
}

// The pass twiddles laid out per (pass, r, k) with k = lane mod ns running
// fastest, for tables staged in LDS: the reads of one pass are unit stride
// (pass 1 reads 4 entries, a broadcast), so they do not conflict on the banks.
//   pass[pass_offset(p) + (r - 1) ns + k] = e^{-2 pi i k r / (4 ns)}, ns = 4^p
//   fold[f]                               = e^{-2 pi i f / 512}
constexpr int kPassTwiddles = 3 * (4 + 16 + 64);
__host__ __device__ __forceinline__ constexpr int pass_offset(int p) {
    return p == 1 ? 0 : (p == 2 ? 3 * 4 : 3 * (4 + 16));
}

// Per lane twiddles of every FFT pass and of the real-FFT fold, loaded once
// per kernel so that no pass waits on a memory load:
//   pass[p][r - 1] = e^{-2 pi i k r / (4 ns)}, ns = 4^p (p = 1..3), k = lane mod ns
//   fold[r]        = e^{-2 pi i f / 512},      f = lane + 64 r
// (pass 0 has ns = 1 and only unit twiddles).
template <typename real>
struct Twiddles {
    using T2 = typename Vec2<real>::type;
    T2 pass[3][3];
    T2 fold[4];

    __device__ __forceinline__ void load(const double2 *tw256, const double2 *tw512, int lane) {
#pragma unroll
        for (int p = 1; p < 4; ++p) {
            const int ns = 1 << (2 * p);
            const int k = lane & (ns - 1);
#pragma unroll
            for (int r = 1; r < 4; ++r)
                pass[p - 1][r - 1] = to_vec2<real>(tw256[(k * r * (64 / ns)) & 255]);
        }
#pragma unroll
        for (int r = 0; r < 4; ++r) fold[r] = to_vec2<real>(tw512[lane + 64 * r]);
    }
    // the same values from the tables kept in the arithmetic's precision
    // (the per pass layout of LdsTwiddles, and the fold's): no conversions
    // for the compiler to place inside the frame loop
    __device__ __forceinline__ void load_staged(const T2 *pass_tab, const T2 *fold_tab, int lane) {
#pragma unroll
        for (int p = 1; p < 4; ++p) {
            const int ns = 1 << (2 * p);
#pragma unroll
            for (int r = 1; r < 4; ++r)
                pass[p - 1][r - 1] = pass_tab[pass_offset(p) + (r - 1) * ns + (lane & (ns - 1))];
        }
#pragma unroll
        for (int r = 0; r < 4; ++r) fold[r] = fold_tab[lane + 64 * r];
    }
    __device__ __forceinline__ T2 pass_tw(int p, int r) const { return pass[p - 1][r - 1]; }
    __device__ __forceinline__ T2 fold_tw(int r) const { return fold[r]; }
};

// The same twiddles read from the tables when a pass needs them: fewer values
// live across the transform, one cached load each.
struct LazyTwiddles {
    const double2 *tw256, *tw512;
    int lane;

    __device__ __forceinline__ double2 pass_tw(int p, int r) const {
        const int ns = 1 << (2 * p);
        const int k = lane & (ns - 1);
        return tw256[(k * r * (64 / ns)) & 255];
    }
    __device__ __forceinline__ double2 fold_tw(int r) const { return tw512[lane + 64 * r]; }
};

// entry i (0 <= i < kPassTwiddles) of the per pass table, from the 256-point table
__host__ __device__ __forceinline__ double2 pass_twiddle_entry(const double2 *tw256, int i) {
    const int p = i < pass_offset(2) ? 1 : (i < pass_offset(3) ? 2 : 3);
    const int ns = 1 << (2 * p);
    const int j = i - pass_offset(p);
    const int r = j / ns + 1, k = j % ns;
    return tw256[(k * r * (64 / ns)) & 255];
}

template <typename real>
struct LdsTwiddles {
    using T2 = typename Vec2<real>::type;
    const T2 *pass, *fold;
    int lane;

    __device__ __forceinline__ T2 pass_tw(int p, int r) const {
        const int ns = 1 << (2 * p);
        return pass[pass_offset(p) + (r - 1) * ns + (lane & (ns - 1))];
    }
    __device__ __forceinline__ T2 fold_tw(int r) const { return fold[lane + 64 * r]; }
};

// In: v[r] = z_{lane + 64 r}.  Out: v[r] = Z_{lane + 64 r} and, with
// kStoreLast, buf[slot(n)] = Z_n (unnormalised; the last pass writes element
// lane + 64 r from lane `lane`, so the lane keeps its own outputs).
template <typename real, bool kInverse, bool kStoreLast = true, class TW>
__device__ __forceinline__ void fft256(cplx<real> (&v)[4], cplx<real> *buf, const TW &tw,
                                       int lane) {
#pragma clang fp contract(off)
#pragma unroll
    for (int pass = 0; pass < 4; ++pass) {
        const int ns = 1 << (2 * pass);
        if (pass > 0) {
#pragma unroll
            for (int r = 0; r < 4; ++r) v[r] = buf[slot(lane + 64 * r)];
            wave_lds_fence();
#pragma unroll
            for (int r = 1; r < 4; ++r) {
                const auto w = tw.pass_tw(pass, r);
                const cplx<real> c = {static_cast<real>(w.x),
                                      static_cast<real>(kInverse ? -w.y : w.y)};
                v[r] = cmul(v[r], c);
            }
        }
        dft4<real, kInverse>(v);
        if (pass == 3 && !kStoreLast) break;
        const int k = lane & (ns - 1);
        const int base = (lane / ns) * ns * 4 + k;
#pragma unroll
        for (int r = 0; r < 4; ++r) buf[slot(base + r * ns)] = v[r];
        wave_lds_fence();
    }
}

// Spectrum of one frame: X_f for f = lane + 64 r (r = 0..3), given the frame
// samples u (already windowed) through the load functor u(k), k < 512.
// tw holds the per lane twiddles (Twiddles::load).  kDoubled returns 2 X_f
// (the fold without its two halvings; scaling by 2 is exact, so a caller that
// takes a factor 1/2 or 1/4 into its own constants gets the same values).
template <typename real, bool kDoubled = false, class Load, class TW>
__device__ __forceinline__ void frame_spectrum(Load u, cplx<real> (&x)[4], cplx<real> *buf,
                                               const TW &tw, int lane) {
#pragma clang fp contract(off)
    cplx<real> v[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) {
        const int n = lane + 64 * r;
        v[r] = {u(2 * n), u(2 * n + 1)};
    }
    fft256<real, false>(v, buf, tw, lane);
#pragma unroll
    for (int r = 0; r < 4; ++r) {
        const int f = lane + 64 * r;
        const cplx<real> zf = v[r];
        const cplx<real> zm = buf[slot((kHalf - f) & (kHalf - 1))];
        // E = (Zf + conj Zm) / 2,  O = -i (Zf - conj Zm) / 2
        const real h = kDoubled ? real(1) : real(0.5);
        const cplx<real> e = {(zf.re + zm.re) * h, (zf.im - zm.im) * h};
        const cplx<real> o = {(zf.im + zm.im) * h, -(zf.re - zm.re) * h};
        const auto w = tw.fold_tw(r);
        const cplx<real> c = {static_cast<real>(w.x), static_cast<real>(w.y)};
        const cplx<real> t = cmul(c, o);
        x[r] = {e.re + t.re, e.im + t.im};
    }
    wave_lds_fence();
}

// Adjoint: given V_f for f = lane + 64 r (zero at f = 0), returns g_u_{2n} and
// g_u_{2n+1} for n = lane + 64 r in (even[r], odd[r]).  V_256 is zero.
template <typename real, class TW>
__device__ __forceinline__ void frame_adjoint(const cplx<real> (&vf)[4], real (&even)[4],
                                              real (&odd)[4], cplx<real> *buf, const TW &tw,
                                              int lane) {
#pragma clang fp contract(off)
#pragma unroll
    for (int r = 0; r < 4; ++r) buf[slot(lane + 64 * r)] = vf[r];
    wave_lds_fence();
    cplx<real> v[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) {
        const int f = lane + 64 * r;
        const cplx<real> a = vf[r];
        // V_{256 - f}; f = 0 pairs with the Nyquist bin, which is zero
        const cplx<real> b = f == 0 ? cplx<real>{real(0), real(0)} : buf[slot(kHalf - f)];
        const cplx<real> s = {a.re + b.re, a.im - b.im};   // V_f + conj V_{256-f}
        const cplx<real> d = {a.re - b.re, a.im + b.im};   // V_f - conj V_{256-f}
        const auto w = tw.fold_tw(r);
        const cplx<real> c = {static_cast<real>(w.x), static_cast<real>(-w.y)};  // e^{+...}
        const cplx<real> t = cmul(c, d);
        // Z' = s + i t
        v[r] = {s.re - t.im, s.im + t.re};
    }
    wave_lds_fence();
    fft256<real, true, false>(v, buf, tw, lane);
#pragma unroll
    for (int r = 0; r < 4; ++r) {
        even[r] = v[r].re;
        odd[r] = v[r].im;
    }
    wave_lds_fence();  // the last pass's reads stay before the caller's next writes
}

}  // namespace pesq
