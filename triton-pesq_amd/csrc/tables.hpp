// Device layout of the constant tables.  Built on the host by
// pesq_model_table_pack / pesq_iir_table_pack (capi.cpp) from the plain C
// structs of pesq_hip.h, copied to device memory by the caller.
#pragma once

#include "iir.hpp"
#include "spectral.hpp"

namespace pesq {

constexpr int kMaxChainBands = 2 * kWave;  // at most two bands per lane

struct ModelTable {
    IirTable iir;                 // A = level alignment band pass, B = pre-emphasis
    double2 tw256[kHalf];         // e^{-2 pi i m / 256}
    double2 tw512[kHalf];         // e^{-2 pi i f / 512}
    // the twiddles in the layouts the STFT kernels stage in LDS, in both
    // arithmetic precisions: per (pass, r, k) (pass_twiddle_entry) and the
    // fold's tw512 in float32
    double2 tw_pass[kPassTwiddles];
    float2 tw_pass_f[kPassTwiddles];
    float2 tw512_f[kHalf];
    float window[kNfft];          // analysis window, centred in n_fft taps
    int32_t band_start[kBands];   // first bin of band i
    int32_t band_end[kBands];     // one past the last bin of band i
    int32_t bin_band[kHalf];      // band owning bin f, -1 if none (bin 0 is -1)
    double corr[kBands];          // power density correction per band
    // per band chain constants (the stand-alone chain takes up to 128 bands)
    double threshs[kMaxChainBands];     // hearing thresholds
    double exps[kMaxChainBands];        // Zwicker exponents
    double loud_scale[kMaxChainBands];  // sl (2 th)^e
    double width[kMaxChainBands];       // band widths in Bark
    double total_width;           // sum of widths of bands 1..
    double sl;                    // loudness calibration constant
    int32_t nbarks;
    int32_t n_fft;
    int32_t hop;
    int32_t pad;
};

// The staged twiddle tables of ModelTable in the arithmetic's precision.
template <typename real>
struct StagedTwiddles;
template <>
struct StagedTwiddles<float> {
    static __device__ __forceinline__ const float2 *pass(const ModelTable &t) { return t.tw_pass_f; }
    static __device__ __forceinline__ const float2 *fold(const ModelTable &t) { return t.tw512_f; }
};
template <>
struct StagedTwiddles<double> {
    static __device__ __forceinline__ const double2 *pass(const ModelTable &t) { return t.tw_pass; }
    static __device__ __forceinline__ const double2 *fold(const ModelTable &t) { return t.tw512; }
};

}  // namespace pesq
