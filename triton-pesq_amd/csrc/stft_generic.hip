// Stand-alone STFT + Bark operator for any power-of-two FFT length and any
// hop (the general TritonStftBark, torch_pesq/triton_ops/spectral.py:584-774):
// n_fft = 32 .. 1024, hop >= 1, up to kGenMaxBands bands of a binary,
// contiguous filterbank.  The PESQ geometry (512 / 256 / 49 bands) has its own
// fused and stand-alone kernels; this file serves every other configuration.
//
// Forward, one wavefront per frame: the real frame u (window applied) is
// folded into the half length complex sequence z_n = u_{2n} + i u_{2n+1},
// transformed by a radix-2 Stockham FFT in a wave-private LDS buffer
// (float64, log2(half) passes, the pass's butterflies spread over the lanes),
// unfolded into X_f, f < half, and |X_f|^2 (DC dropped) summed per band.
//
// Backward: the same spectrum per frame, V_f = g_P(f) X_f, the adjoint of the
// fold and an inverse FFT give the frame's sample gradient, which is written
// (times the window) to a [rows, frames, n_fft] scratch; a gather kernel then
// adds, for each sample, the contributions of the frames that cover it in
// increasing frame order (deterministic, no atomics, any hop including hops
// longer than n_fft, whose uncovered samples get exactly zero).
#include <cmath>
#include <cstring>

#include "common.hpp"
#include "spectral.hpp"

namespace pesq {

constexpr int kGenMaxHalf = 512;   // n_fft <= 1024
constexpr int kGenMinHalf = 16;    // n_fft >= 32
constexpr int kGenMaxBands = 128;
constexpr int kGenPerLane = kGenMaxHalf / kWave;       // points per lane (<= 8)
constexpr int kGenBfly = kGenMaxHalf / 2 / kWave;      // butterflies per lane (<= 4)
constexpr int kGenWaves = 4;                           // frames per workgroup

struct StftTable {
    int32_t n_fft, half, hop, nbarks;
    double2 tw[kGenMaxHalf / 2];      // e^{-2 pi i m / half}, m < half / 2
    double2 fold[kGenMaxHalf];        // e^{-2 pi i f / n_fft}, f < half
    float window[2 * kGenMaxHalf];    // n_fft taps, centred
    int32_t band_start[kGenMaxBands];
    int32_t band_end[kGenMaxBands];
    int32_t bin_band[kGenMaxHalf];    // band of bin f, -1 for none and for f = 0
    double corr[kGenMaxBands];
};

struct GenArgs {
    const StftTable *tab;
    const float *x;       // [rows, len]
    float *bark;          // [rows, frames, nbarks]
    const float *gbark;   // [rows, frames, nbarks]
    float *gx;            // [rows, len]
    float *scratch;       // [rows, frames, n_fft]
    int64_t rows, len, frames, ftiles;
    int n_fft, half, hop, nbarks;
};

using c64g = cplx<double>;

// In place radix-2 Stockham FFT of buf[0 .. half) (natural order in and out),
// e^{-2 pi i / half} forward, conjugate twiddles for the inverse; unnormalised.
// Pass s (sub-transform size ns = 2^s): butterfly j takes buf[j] and
// buf[j + half / 2], k = j mod ns, w = e^{-2 pi i k / (2 ns)}, and writes
// positions (j / ns) 2 ns + k and that plus ns.  Every lane reads all of its
// butterflies' inputs before the wave's writes start.
template <bool kInv>
__device__ __forceinline__ void gen_fft(c64g *buf, const double2 *tw, int half, int lane) {
    const int nb = half / 2;
    for (int ns = 1; ns < half; ns *= 2) {
        c64g a[kGenBfly], b[kGenBfly];
#pragma unroll
        for (int q = 0; q < kGenBfly; ++q) {
            const int j = lane + kWave * q;
            if (j < nb) {
                a[q] = buf[j];
                b[q] = buf[j + nb];
            }
        }
        wave_lds_fence();
#pragma unroll
        for (int q = 0; q < kGenBfly; ++q) {
            const int j = lane + kWave * q;
            if (j < nb) {
                const int k = j & (ns - 1);
                const double2 w = tw[k * (nb / ns)];
                const c64g v = cmul(b[q], c64g{w.x, kInv ? -w.y : w.y});
                const int o = (j / ns) * 2 * ns + k;
                buf[o] = {a[q].re + v.re, a[q].im + v.im};
                buf[o + ns] = {a[q].re - v.re, a[q].im - v.im};
            }
        }
        wave_lds_fence();
    }
}

// spectrum X_f, f = lane + 64 r < half, of the frame starting at `start`;
// buf ends up holding Z (the half length transform)
__device__ __forceinline__ void gen_spectrum(const StftTable &t, const float *x, int64_t start,
                                             int64_t len, int half, c64g *buf, int lane,
                                             c64g (&spec)[kGenPerLane]) {
#pragma unroll
    for (int r = 0; r < kGenPerLane; ++r) {
        const int n = lane + kWave * r;
        if (n < half) {
            const double u0 = static_cast<double>(load_or_zero(x, start + 2 * n, len)) *
                              static_cast<double>(t.window[2 * n]);
            const double u1 = static_cast<double>(load_or_zero(x, start + 2 * n + 1, len)) *
                              static_cast<double>(t.window[2 * n + 1]);
            buf[n] = {u0, u1};
        }
    }
    wave_lds_fence();
    gen_fft<false>(buf, t.tw, half, lane);
#pragma unroll
    for (int r = 0; r < kGenPerLane; ++r) {
        const int f = lane + kWave * r;
        if (f < half) {
            const c64g zf = buf[f];
            const c64g zm = buf[(half - f) & (half - 1)];
            const c64g e = {(zf.re + zm.re) * 0.5, (zf.im - zm.im) * 0.5};
            const c64g o = {(zf.im + zm.im) * 0.5, -(zf.re - zm.re) * 0.5};
            const double2 c = t.fold[f];
            const c64g v = cmul(c64g{c.x, c.y}, o);
            spec[r] = {e.re + v.re, e.im + v.im};
        }
    }
    wave_lds_fence();
}

__global__ void __launch_bounds__(kWave *kGenWaves) stft_gen_fwd_kernel(GenArgs a) {
    __shared__ c64g bufs[kGenWaves][kGenMaxHalf];
    const StftTable &t = *a.tab;
    const int64_t row = blockIdx.x / a.ftiles;
    const int64_t ft = blockIdx.x - row * a.ftiles;
    const int wave = threadIdx.x / kWave;
    const int lane = threadIdx.x % kWave;
    const int64_t frame = ft * kGenWaves + wave;
    if (frame >= a.frames) return;  // whole wavefronts; no block barrier follows
    c64g *buf = bufs[wave];
    c64g spec[kGenPerLane];
    gen_spectrum(t, a.x + row * a.len, frame * a.hop, a.len, a.half, buf, lane, spec);
    double *power = reinterpret_cast<double *>(buf);
#pragma unroll
    for (int r = 0; r < kGenPerLane; ++r) {
        const int f = lane + kWave * r;
        if (f < a.half) power[f] = f == 0 ? 0.0 : spec[r].re * spec[r].re + spec[r].im * spec[r].im;
    }
    wave_lds_fence();
    float *out = a.bark + (row * a.frames + frame) * a.nbarks;
    for (int b = lane; b < a.nbarks; b += kWave) {
        double acc = 0.0;
        for (int f = t.band_start[b]; f < t.band_end[b]; ++f) acc += power[f];
        out[b] = static_cast<float>(acc * t.corr[b]);
    }
}

// per frame: the frame's windowed sample gradient into the scratch
__global__ void __launch_bounds__(kWave *kGenWaves) stft_gen_bwd_frames_kernel(GenArgs a) {
    __shared__ c64g bufs[kGenWaves][kGenMaxHalf];
    __shared__ float gband[kGenWaves][kGenMaxBands];
    const StftTable &t = *a.tab;
    const int64_t row = blockIdx.x / a.ftiles;
    const int64_t ft = blockIdx.x - row * a.ftiles;
    const int wave = threadIdx.x / kWave;
    const int lane = threadIdx.x % kWave;
    const int64_t frame = ft * kGenWaves + wave;
    if (frame >= a.frames) return;
    const int half = a.half;
    const float *g = a.gbark + (row * a.frames + frame) * a.nbarks;
    for (int b = lane; b < a.nbarks; b += kWave) {
        gband[wave][b] = static_cast<float>(static_cast<double>(g[b]) * t.corr[b]);
    }
    c64g *buf = bufs[wave];
    c64g spec[kGenPerLane];
    gen_spectrum(t, a.x + row * a.len, frame * a.hop, a.len, half, buf, lane, spec);
    // V_f = g_P(f) X_f (zero at DC and outside the bands), staged for V_{half - f}
#pragma unroll
    for (int r = 0; r < kGenPerLane; ++r) {
        const int f = lane + kWave * r;
        if (f < half) {
            const int band = t.bin_band[f];
            const double gp = band >= 0 ? static_cast<double>(gband[wave][band]) : 0.0;
            spec[r] = {gp * spec[r].re, gp * spec[r].im};
            buf[f] = spec[r];
        }
    }
    wave_lds_fence();
    // Z'_f = (V_f + conj V_{half-f}) + i e^{+2 pi i f / n} (V_f - conj V_{half-f}), V_half = 0
    c64g zp[kGenPerLane];
#pragma unroll
    for (int r = 0; r < kGenPerLane; ++r) {
        const int f = lane + kWave * r;
        if (f < half) {
            const c64g va = spec[r];
            const c64g vb = f == 0 ? c64g{0.0, 0.0} : buf[half - f];
            const c64g s = {va.re + vb.re, va.im - vb.im};
            const c64g d = {va.re - vb.re, va.im + vb.im};
            const double2 c = t.fold[f];
            const c64g v = cmul(c64g{c.x, -c.y}, d);
            zp[r] = {s.re - v.im, s.im + v.re};
        }
    }
    wave_lds_fence();
#pragma unroll
    for (int r = 0; r < kGenPerLane; ++r) {
        const int f = lane + kWave * r;
        if (f < half) buf[f] = zp[r];
    }
    wave_lds_fence();
    gen_fft<true>(buf, t.tw, half, lane);
    float *dst = a.scratch + (row * a.frames + frame) * a.n_fft;
#pragma unroll
    for (int r = 0; r < kGenPerLane; ++r) {
        const int n = lane + kWave * r;
        if (n < half) {
            const c64g z = buf[n];
            dst[2 * n] = static_cast<float>(z.re * static_cast<double>(t.window[2 * n]));
            dst[2 * n + 1] = static_cast<float>(z.im * static_cast<double>(t.window[2 * n + 1]));
        }
    }
}

constexpr int kGatherThreads = 256;

// per sample: sum of the contributions of the frames covering it, in
// increasing frame order
__global__ void __launch_bounds__(kGatherThreads) stft_gen_bwd_gather_kernel(GenArgs a) {
    const int64_t nblk = cdiv(a.len, kGatherThreads);
    const int64_t row = blockIdx.x / nblk;
    const int64_t n = (blockIdx.x - row * nblk) * kGatherThreads + threadIdx.x;
    if (n >= a.len) return;
    // frames t with t hop <= n < t hop + n_fft, t < frames
    const int64_t t_lo = n < a.n_fft ? 0 : (n - a.n_fft) / a.hop + 1;
    int64_t t_hi = n / a.hop;
    if (t_hi > a.frames - 1) t_hi = a.frames - 1;
    const float *src = a.scratch + row * a.frames * a.n_fft;
    double g = 0.0;
    for (int64_t t = t_lo; t <= t_hi; ++t) g += static_cast<double>(src[t * a.n_fft + (n - t * a.hop)]);
    a.gx[row * a.len + n] = static_cast<float>(g);
}

static int check_geometry(int64_t rows, int64_t len, int64_t n_padded, int n_fft, int hop,
                          int nbarks, int64_t &frames) {
    PESQ_CHECK_ARG(rows >= 0 && len >= 0, "invalid sizes");
    PESQ_CHECK_ARG(n_fft >= 2 * kGenMinHalf && n_fft <= 2 * kGenMaxHalf && (n_fft & (n_fft - 1)) == 0,
                   "n_fft has to be a power of two in [%d, %d], got %d", 2 * kGenMinHalf,
                   2 * kGenMaxHalf, n_fft);
    PESQ_CHECK_ARG(hop >= 1, "hop_length has to be positive, got %d", hop);
    PESQ_CHECK_ARG(nbarks >= 1 && nbarks <= kGenMaxBands, "1..%d bands, got %d", kGenMaxBands,
                   nbarks);
    PESQ_CHECK_ARG(n_padded >= len && n_padded >= n_fft,
                   "n_padded (%lld) has to cover the signal (%lld) and one frame (%d)",
                   (long long)n_padded, (long long)len, n_fft);
    frames = 1 + (n_padded - n_fft) / hop;
    PESQ_CHECK_ARG(rows * cdiv(frames, kGenWaves) < (int64_t(1) << 31) &&
                       rows * cdiv(len, kGatherThreads) < (int64_t(1) << 31),
                   "problem too large for one launch");
    return PESQ_OK;
}

}  // namespace pesq

using namespace pesq;

extern "C" size_t pesq_stft_table_bytes(void) { return sizeof(StftTable); }

extern "C" int pesq_stft_table_pack(int n_fft, int hop, const float *window, int nbarks,
                                    const int32_t *band_start, const int32_t *band_end,
                                    const double *corr, void *out) {
    PESQ_CHECK_ARG(window && band_start && band_end && corr && out, "null argument");
    int64_t frames = 0;
    if (int st = check_geometry(0, 0, n_fft, n_fft, hop, nbarks, frames)) return st;
    StftTable *t = new StftTable;
    std::memset(t, 0, sizeof(*t));
    const int half = n_fft / 2;
    t->n_fft = n_fft;
    t->half = half;
    t->hop = hop;
    t->nbarks = nbarks;
    const double two_pi = 6.283185307179586476925286766559;
    for (int m = 0; m < half / 2; ++m) {
        t->tw[m] = make_double2(std::cos(two_pi * m / half), -std::sin(two_pi * m / half));
    }
    for (int f = 0; f < half; ++f) {
        t->fold[f] = make_double2(std::cos(two_pi * f / n_fft), -std::sin(two_pi * f / n_fft));
        t->bin_band[f] = -1;
    }
    std::memcpy(t->window, window, sizeof(float) * n_fft);
    int prev = 0;
    for (int b = 0; b < nbarks; ++b) {
        const int lo = band_start[b], hi = band_end[b];
        if (lo < prev || hi < lo || hi > half) {
            delete t;
            set_error("Bark band %d covers [%d, %d): bands must be sorted, disjoint and inside "
                      "[0, %d)", b, lo, hi, half);
            return PESQ_ERR_ARGUMENT;
        }
        t->band_start[b] = lo;
        t->band_end[b] = hi;
        t->corr[b] = corr[b];
        for (int f = lo; f < hi; ++f) t->bin_band[f] = b;
        prev = hi;
    }
    t->bin_band[0] = -1;  // the DC bin is dropped
    std::memcpy(out, t, sizeof(*t));
    delete t;
    return PESQ_OK;
}

extern "C" int pesq_stft_workspace(int64_t rows, int64_t len, int64_t n_padded, int n_fft,
                                   int hop, size_t *bytes) {
    PESQ_CHECK_ARG(bytes != nullptr, "null argument");
    int64_t frames = 0;
    if (int st = check_geometry(rows, len, n_padded, n_fft, hop, 1, frames)) return st;
    *bytes = size_t(rows) * size_t(frames) * size_t(n_fft) * sizeof(float);
    return PESQ_OK;
}

extern "C" int pesq_stft_forward(const float *x, int64_t rows, int64_t len, int64_t n_padded,
                                 const void *table, int n_fft, int hop, int nbarks, float *bark,
                                 hipStream_t stream) {
    PESQ_CHECK_ARG(x && table && bark, "null pointer argument");
    GenArgs a{};
    int64_t frames = 0;
    if (int st = check_geometry(rows, len, n_padded, n_fft, hop, nbarks, frames)) return st;
    if (rows == 0) return PESQ_OK;
    PESQ_CHECK_ARG(len > 0, "empty signal with frames to fill");
    a.tab = static_cast<const StftTable *>(table);
    a.x = x;
    a.bark = bark;
    a.rows = rows;
    a.len = len;
    a.frames = frames;
    a.ftiles = cdiv(frames, kGenWaves);
    a.n_fft = n_fft;
    a.half = n_fft / 2;
    a.hop = hop;
    a.nbarks = nbarks;
    hipLaunchKernelGGL(stft_gen_fwd_kernel, dim3(static_cast<unsigned>(rows * a.ftiles)),
                       dim3(kWave * kGenWaves), 0, stream, a);
    PESQ_CHECK_LAUNCH("stft forward");
    return PESQ_OK;
}

extern "C" int pesq_stft_backward(const float *gbark, const float *x, int64_t rows, int64_t len,
                                  int64_t n_padded, const void *table, int n_fft, int hop,
                                  int nbarks, float *gx, void *workspace, hipStream_t stream) {
    PESQ_CHECK_ARG(gbark && x && table && gx && workspace, "null pointer argument");
    GenArgs a{};
    int64_t frames = 0;
    if (int st = check_geometry(rows, len, n_padded, n_fft, hop, nbarks, frames)) return st;
    if (rows == 0 || len == 0) return PESQ_OK;
    a.tab = static_cast<const StftTable *>(table);
    a.x = x;
    a.gbark = gbark;
    a.gx = gx;
    a.scratch = static_cast<float *>(workspace);
    a.rows = rows;
    a.len = len;
    a.frames = frames;
    a.ftiles = cdiv(frames, kGenWaves);
    a.n_fft = n_fft;
    a.half = n_fft / 2;
    a.hop = hop;
    a.nbarks = nbarks;
    hipLaunchKernelGGL(stft_gen_bwd_frames_kernel, dim3(static_cast<unsigned>(rows * a.ftiles)),
                       dim3(kWave * kGenWaves), 0, stream, a);
    PESQ_CHECK_LAUNCH("stft backward frames");
    hipLaunchKernelGGL(stft_gen_bwd_gather_kernel,
                       dim3(static_cast<unsigned>(rows * cdiv(len, kGatherThreads))),
                       dim3(kGatherThreads), 0, stream, a);
    PESQ_CHECK_LAUNCH("stft backward gather");
    return PESQ_OK;
}
