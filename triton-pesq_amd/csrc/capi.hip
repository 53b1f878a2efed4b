// Host side of the C ABI: error reporting and constant table packing.
#include <cmath>
#include <cstdarg>
#include <cstring>

#include "tables.hpp"

namespace pesq {

static thread_local char g_error[512] = "";

void set_error(const char *fmt, ...) {
    va_list args;
    va_start(args, fmt);
    std::vsnprintf(g_error, sizeof(g_error), fmt, args);
    va_end(args);
}

// A^n for the 2x2 companion block [[-a1, 1], [-a2, 0]], fp64
static void mat_mul(const double *x, const double *y, double *out) {
    const double r0 = x[0] * y[0] + x[1] * y[2];
    const double r1 = x[0] * y[1] + x[1] * y[3];
    const double r2 = x[2] * y[0] + x[3] * y[2];
    const double r3 = x[2] * y[1] + x[3] * y[3];
    out[0] = r0;
    out[1] = r1;
    out[2] = r2;
    out[3] = r3;
}

// Sections are stored with b2 = 0: a section with b2 != 0 and a2 != 0 is
// rewritten as the direct term b2 / a2 plus the section
// (b0 - b2 / a2) + (b1 - a1 b2 / a2) z^-1 over the same denominator, which is
// the same transfer function.  `direct` accumulates the direct terms.
// Section coefficients and scan powers of s into table sections first.. of t.
// With fold_b2 (parallel form) a section's b2 becomes the direct term b2/a2
// plus a section without z^-2 in its numerator; otherwise b2 is kept (the
// full biquads of a cascade).
static int fill_sections(IirTable &t, int first, const pesq_iir_sections &s, double &direct,
                         bool fold_b2 = true) {
    PESQ_CHECK_ARG(s.count >= 1 && first + s.count <= kMaxSections,
                   "an IIR filter needs 1..%d sections in total, got %d", kMaxSections,
                   first + s.count);
    for (int k = 0; k < s.count; ++k) {
        const int q = first + k;
        PESQ_CHECK_ARG(std::isfinite(s.b0[k]) && std::isfinite(s.b1[k]) && std::isfinite(s.b2[k]) &&
                           std::isfinite(s.a1[k]) && std::isfinite(s.a2[k]),
                       "non finite IIR coefficient in section %d", k);
        PESQ_CHECK_ARG(!fold_b2 || s.b2[k] == 0.0 || s.a2[k] != 0.0,
                       "section %d has b2 != 0 over a first order denominator (an FIR tail)", k);
        const double d = (!fold_b2 || s.b2[k] == 0.0) ? 0.0 : s.b2[k] / s.a2[k];
        direct += d;
        t.b0[q] = s.b0[k] - d;
        t.b1[q] = s.b1[k] - s.a1[k] * d;
        t.b2[q] = fold_b2 ? 0.0 : s.b2[k];
        t.a1[q] = s.a1[k];
        t.a2[q] = s.a2[k];
        // chunk transfer powers: level 0 = A^kChunk, level j = A^(kChunk 2^j)
        const double a[4] = {-s.a1[k], 1.0, -s.a2[k], 0.0};
        double p[4] = {1.0, 0.0, 0.0, 1.0};
        for (int i = 0; i < kChunk; ++i) mat_mul(a, p, p);
        for (int level = 0; level < kLevels; ++level) {
            std::memcpy(t.pw[level][q], p, sizeof(p));
            mat_mul(p, p, p);
        }
        // chunk end state weights: fir[i] = A^(kChunk - 1 - i) beta, beta the
        // state increment per unit input (y = b0 x + z1 feeds back through a1, a2)
        {
            double g[2] = {t.b1[q] - s.a1[k] * t.b0[q], t.b2[q] - s.a2[k] * t.b0[q]};
            for (int m = 0; m < kChunk; ++m) {
                t.fir[q][kChunk - 1 - m][0] = g[0];
                t.fir[q][kChunk - 1 - m][1] = g[1];
                const double g0 = a[0] * g[0] + a[1] * g[1];
                const double g1 = a[2] * g[0] + a[3] * g[1];
                g[0] = g0;
                g[1] = g1;
            }
        }
        // block pair powers M^(2 i), M = A^kSpan (level kLevelBlock)
        {
            double m[4] = {1.0, 0.0, 0.0, 1.0};
            for (int i = 0; i < kWave; ++i) {
                std::memcpy(t.blk_pw2[i][q], m, sizeof(m));
                mat_mul(t.pw[kLevelBlock + 1][q], m, m);
            }
        }
        // lane start powers A^(kChunk lane): product of the levels of the set bits
        for (int lane = 0; lane < kWave; ++lane) {
            double m[4] = {1.0, 0.0, 0.0, 1.0};
            for (int level = 0; level < kLevelBlock; ++level) {
                if (lane & (1 << level)) mat_mul(t.pw[level][q], m, m);
            }
            std::memcpy(t.lane_pw[q][lane], m, sizeof(m));
        }
    }
    return PESQ_OK;
}

static int pack_iir(IirTable &t, const pesq_iir_sections *a, const pesq_iir_sections *b) {
    std::memset(&t, 0, sizeof(t));
    PESQ_CHECK_ARG(a != nullptr, "null filter");
    t.na = a->count;
    t.nb = b ? b->count : 0;
    t.c0a = a->c0;
    t.c0b = b ? b->c0 : 0.0;
    if (int st = fill_sections(t, 0, *a, t.c0a)) return st;
    if (b) {
        if (int st = fill_sections(t, a->count, *b, t.c0b)) return st;
    }
    return PESQ_OK;
}

}  // namespace pesq

using namespace pesq;

extern "C" int pesq_abi_version(void) { return 2; }

extern "C" const char *pesq_last_error(void) { return g_error; }

extern "C" size_t pesq_iir_table_bytes(void) { return sizeof(IirTable); }

extern "C" int pesq_iir_table_pack(const pesq_iir_sections *filter, void *out) {
    PESQ_CHECK_ARG(out != nullptr, "null output buffer");
    IirTable t;
    if (int st = pack_iir(t, filter, nullptr)) return st;
    std::memcpy(out, &t, sizeof(t));
    return PESQ_OK;
}

extern "C" int pesq_iir_cascade_pack(const double *sos, int sections, void *out) {
    PESQ_CHECK_ARG(sos != nullptr && out != nullptr, "null argument");
    PESQ_CHECK_ARG(sections >= 1 && sections <= PESQ_IIR_MAX_CASCADE,
                   "a cascade has 1..%d sections, got %d", PESQ_IIR_MAX_CASCADE, sections);
    IirTable *tables = static_cast<IirTable *>(out);
    for (int k = 0; k < sections; ++k) {
        const double *row = sos + 6 * k;
        PESQ_CHECK_ARG(row[3] != 0.0 && std::isfinite(row[3]),
                       "section %d has a zero leading denominator coefficient", k);
        pesq_iir_sections one{};
        one.count = 1;
        one.b0[0] = row[0] / row[3];
        one.b1[0] = row[1] / row[3];
        one.b2[0] = row[2] / row[3];
        one.a1[0] = row[4] / row[3];
        one.a2[0] = row[5] / row[3];
        IirTable t;
        std::memset(&t, 0, sizeof(t));
        t.na = 1;
        if (int st = fill_sections(t, 0, one, t.c0a, false)) return st;
        std::memcpy(&tables[k], &t, sizeof(t));
    }
    return PESQ_OK;
}

extern "C" size_t pesq_model_table_bytes(void) { return sizeof(ModelTable); }

extern "C" int pesq_chain_table_pack(int nbands, const double *threshs, const double *exps,
                                     const double *widths, double total_width, double sl,
                                     void *out) {
    PESQ_CHECK_ARG(threshs && exps && widths && out, "null argument");
    PESQ_CHECK_ARG(nbands >= 1 && nbands <= kMaxChainBands, "the chain takes 1 .. %d bands, got %d",
                   kMaxChainBands, nbands);
    ModelTable *t = new ModelTable;
    std::memset(t, 0, sizeof(*t));
    for (int i = 0; i < nbands; ++i) {
        if (!(threshs[i] > 0.0) || !std::isfinite(exps[i]) || !std::isfinite(widths[i])) {
            delete t;
            set_error("Hearing thresholds have to be strictly positive (band %d).", i);
            return PESQ_ERR_ARGUMENT;
        }
        t->threshs[i] = threshs[i];
        t->exps[i] = exps[i];
        t->width[i] = widths[i];
        t->loud_scale[i] = sl * std::pow(2.0 * threshs[i], exps[i]);
    }
    t->total_width = total_width;
    t->sl = sl;
    t->nbarks = nbands;
    std::memcpy(out, t, sizeof(*t));
    delete t;
    return PESQ_OK;
}

extern "C" int pesq_model_table_pack(const pesq_model_constants *c, void *out) {
    PESQ_CHECK_ARG(c != nullptr && out != nullptr, "null argument");
    PESQ_CHECK_ARG(c->nbarks == kBands && c->n_fft == kNfft && c->hop == kHop,
                   "the HIP pipeline supports nbarks=49, n_fft=512, hop_length=256 "
                   "(got %d, %d, %d)",
                   c->nbarks, c->n_fft, c->hop);
    const bool no_filters = c->power_filter.count == 0 && c->pre_filter.count == 0;
    PESQ_CHECK_ARG(no_filters || (c->power_filter.count == 5 && c->pre_filter.count == 1),
                   "the HIP pipeline is built for a 5 section level alignment filter and a "
                   "1 section pre-emphasis filter (got %d and %d)",
                   c->power_filter.count, c->pre_filter.count);

    ModelTable *t = new ModelTable;
    std::memset(t, 0, sizeof(*t));
    if (!no_filters) {
        const int st = pack_iir(t->iir, &c->power_filter, &c->pre_filter);
        if (st) {
            delete t;
            return st;
        }
        // the pipeline's scans start every block from the two blocks before
        // it, run from a zero state (iir.hpp, windowed block starts): every
        // section's state must have decayed below kWindowDecay over that span
        for (int q = 0; q < t->iir.na + t->iir.nb; ++q) {
            double m[4] = {1.0, 0.0, 0.0, 1.0};
            for (int w = 0; w < kWarmBlocks; ++w) mat_mul(t->iir.pw[kLevelBlock][q], m, m);
            double mx = 0.0;
            for (double v : m) mx = std::fmax(mx, std::fabs(v));
            if (!(mx <= kWindowDecay)) {
                const char *name = q < t->iir.na ? "level alignment" : "pre-emphasis";
                set_error("the %s filter decays too slowly for the pipeline: section %d keeps "
                          "%.3g of its state over %d samples (at most %.0e)",
                          name, q, mx, kWarmBlocks * kSpan, kWindowDecay);
                delete t;
                return PESQ_ERR_ARGUMENT;
            }
        }
    }

    const double two_pi = 6.283185307179586476925286766559;
    for (int m = 0; m < kHalf; ++m) {
        t->tw256[m] = make_double2(std::cos(two_pi * m / 256.0), -std::sin(two_pi * m / 256.0));
        t->tw512[m] = make_double2(std::cos(two_pi * m / 512.0), -std::sin(two_pi * m / 512.0));
        t->tw512_f[m] = make_float2(static_cast<float>(t->tw512[m].x),
                                    static_cast<float>(t->tw512[m].y));
    }
    for (int i = 0; i < kPassTwiddles; ++i) {
        t->tw_pass[i] = pass_twiddle_entry(t->tw256, i);
        t->tw_pass_f[i] = make_float2(static_cast<float>(t->tw_pass[i].x),
                                      static_cast<float>(t->tw_pass[i].y));
    }
    std::memcpy(t->window, c->window, sizeof(t->window));

    for (int f = 0; f < kHalf; ++f) t->bin_band[f] = -1;
    int prev = 0;
    for (int i = 0; i < kBands; ++i) {
        const int lo = c->band_start[i], hi = c->band_end[i];
        if (lo < prev || hi < lo || hi > kHalf || hi - lo > kMaxBandBins) {
            delete t;
            set_error("Bark band %d covers [%d, %d): bands must be sorted, disjoint, "
                      "inside [0, 256) and at most %d bins wide",
                      i, lo, hi, kMaxBandBins);
            return PESQ_ERR_ARGUMENT;
        }
        t->band_start[i] = lo;
        t->band_end[i] = hi;
        for (int f = lo; f < hi; ++f) t->bin_band[f] = i;
        prev = hi;
        if (!(c->threshs[i] > 0.0)) {
            delete t;
            set_error("Hearing thresholds have to be strictly positive.");
            return PESQ_ERR_ARGUMENT;
        }
        t->corr[i] = c->corr[i];
        t->threshs[i] = c->threshs[i];
        t->exps[i] = c->exps[i];
        t->width[i] = c->width[i];
        t->loud_scale[i] = c->sl * std::pow(2.0 * c->threshs[i], c->exps[i]);
    }
    // the DC bin is dropped (the energy feature is unused)
    t->bin_band[0] = -1;
    t->total_width = c->total_width;
    t->sl = c->sl;
    t->nbarks = kBands;
    t->n_fft = kNfft;
    t->hop = kHop;

    std::memcpy(out, t, sizeof(*t));
    delete t;
    return PESQ_OK;
}
