// Workspace layout of the fused pipeline (host and device agree on it).
#pragma once

#include <cstring>

#include "common.hpp"
#include "iir.hpp"
#include "spectral.hpp"

namespace pesq {

constexpr int kPowerSections = 5;  // order 10 band pass, parallel form
constexpr int kPreSections = 1;    // pre-emphasis biquad
constexpr int kPipeSections = kPowerSections + kPreSections;  // scanned in one pass
#ifndef PESQ_WINDOW_STARTS
#define PESQ_WINDOW_STARTS 1
#endif
// The pipeline's filters decay below kWindowDecay over kWarmBlocks blocks
// (pesq_model_table_pack rejects tables whose filters do not), so its scans
// on lane-state grids take windowed block starts (kWindowStarts) and have no
// prefix pass.
constexpr bool kPipeWindow = PESQ_WINDOW_STARTS != 0;
constexpr int kTile = 16;          // frames per workgroup of the STFT / chain kernels
constexpr int kBwdFrames = 8;      // frames per workgroup of the plain STFT backward
constexpr int kBwdHops = kBwdFrames - 1;  // output hop blocks per such workgroup
constexpr int kBwdWaves = 8;       // wavefronts per workgroup of the fused STFT backward (large grids)
#ifndef PESQ_BWD_WAVES_SMALL
#define PESQ_BWD_WAVES_SMALL 9
#endif
constexpr int kBwdWavesSmall = PESQ_BWD_WAVES_SMALL;  // and of small grids (one frame each)
// Grids of more chain tiles (batch x ntile) than this are throughput bound:
// the kernels take their wide variants (more frames per wavefront).
#ifndef PESQ_WIDE_TILES
#define PESQ_WIDE_TILES 512
#endif
constexpr int64_t kWideTiles = PESQ_WIDE_TILES;
// Items of more chain tiles than this sum their per tile band partials once
// per item (band_totals_kernel) instead of in every workgroup that reads them
// (the chain forward's and the STFT backward's, whose reads then grow with
// the square of the item length).
constexpr int64_t kTotalsTiles = 64;
constexpr int kWin = 20;           // PSQM window (frames)
constexpr int kStride = 10;        // PSQM stride (frames)

// per frame chain arrays, [batch, frames] each
enum FrameArray { kTaer, kTad, kFpr0, kFpr1, kH, kSymmRaw, kAsymmRaw, kSymm, kAsymm, kFrameArrays };
// per band chain arrays, [batch, bands] each
enum BandArray { kR, kRatio, kMref, kBandArrays };
// per (frame, band) terms of the forward chain that the backward reads,
// [batch, frames, bands] of float4 (ChainTerms in pipeline.hip): the clamped
// disturbance, the asymmetry factor with its clamp state, and the slopes of
// both loudnesses
constexpr size_t kChainTermBytes = 16;

struct PipeLayout {
    int64_t batch = 0, len = 0, rows = 0, frames = 0;
    int64_t nblk = 0, ntile = 0, nhoptile = 0, nhop = 0, nwin = 0;
    int64_t row0 = 0, nrg = 0;  // stacked rows that receive gradients
    int grad_mask = 0;
    int nb = kBands;            // Bark bands (the stand-alone chain takes 1 .. 128)
    int loud_store = 0;         // the forward writes the `loud` region (a backward follows)
    int bwd_fpw = 1;            // frames per wavefront of the fused STFT backward (1 or 2)
    int bwd_waves = kBwdWaves;  // wavefronts per workgroup of the fused STFT backward
    int totals = 0;             // per item band totals (items of more than kTotalsTiles tiles)
    // The forward's STFT kernel also runs the aggregate pass of the backward's
    // level alignment filter (power^T on f, which only needs forward data), on
    // grids whose backward scan stores lane states, with rows of up to
    // kFusedPrefixBlocks blocks and up to kWideTiles chain tiles (the STFT
    // forward's variant for more tiles keeps its lean register budget);
    // the backward's output launch then warms the pre-emphasis filter's block
    // start states up from the two previous blocks, and there is no aggregate launch.
    // The backward scan's workspace (aggr_b) then lies in the forward workspace.
    int host_power = 0;

    // forward workspace
    size_t aggr = 0, energy = 0, p = 0, f = 0, rowconst = 0, bark = 0, keep = 0;
    size_t bandref = 0, banddeg = 0, frame = 0, band = 0, psqm = 0, dist = 0, loud = 0;
    size_t bandtot = 0;  // [batch, 2, nb] totals of bandref, banddeg (with `totals`)
    size_t fwd_bytes = 0;
    // backward workspace
    size_t gbark = 0, grpart = 0, gp = 0, spart = 0, aggr_b = 0, bwd_bytes = 0;
    size_t gradtot = 0;  // [batch, nb] totals of grpart (with `totals`)

    static size_t align(size_t v) { return (v + 255) & ~size_t(255); }

    static int64_t frames_for(int64_t len) {
        const int64_t padded = len + len % 256;
        return padded < kNfft ? 0 : 1 + (padded - kNfft) / kHop;
    }

    void build(int64_t b, int64_t n, int mask) {
        nb = kBands;
        batch = b;
        len = n;
        rows = 2 * b;
        grad_mask = mask;
        frames = frames_for(n);
        nblk = cdiv(n, kBlockSpan);
        ntile = cdiv(frames, kTile);
        bwd_fpw = b * ntile > kWideTiles ? 2 : 1;
        totals = ntile > kTotalsTiles;
        bwd_waves = bwd_fpw == 2 ? kBwdWaves : kBwdWavesSmall;
        nhop = cdiv(n, kHop);
        nhoptile = cdiv(nhop, bwd_waves * bwd_fpw - 1);
        nwin = frames >= kWin ? (frames - kWin) / kStride + 1 : 0;
        row0 = (mask & PESQ_GRAD_REF) ? 0 : b;
        nrg = mask == (PESQ_GRAD_REF | PESQ_GRAD_DEG) ? 2 * b : (mask ? b : 0);

        size_t off = 0;
        auto take = [&](size_t &field, size_t bytes) {
            field = off;
            off = align(off + bytes);
        };
        take(aggr, size_t(scan_workspace_doubles(rows, nblk, kPipeSections)) * sizeof(double));
        take(energy, size_t(rows) * nblk * sizeof(double));
        take(p, size_t(rows) * len * sizeof(float));
        take(f, size_t(nrg) * len * sizeof(float));
        take(rowconst, size_t(rows) * 4 * sizeof(double));
        take(bark, size_t(rows) * frames * nb * sizeof(float));
        take(keep, size_t(batch) * frames * sizeof(float));
        take(bandref, size_t(batch) * ntile * nb * sizeof(double));
        take(banddeg, size_t(batch) * ntile * nb * sizeof(double));
        take(frame, size_t(kFrameArrays) * batch * frames * sizeof(double));
        take(band, size_t(kBandArrays) * batch * nb * sizeof(double));
        take(psqm, size_t(2) * batch * nwin * sizeof(double));
        take(dist, size_t(batch) * 2 * sizeof(double));
        loud_store = mask != 0;
        take(loud, loud_store ? kChainTermBytes * batch * frames * nb : 0);
        take(bandtot, totals ? size_t(2) * batch * nb * sizeof(double) : 0);
        const ScanPlan bwd_scan = scan_plan(nrg, nblk);
        host_power = nrg > 0 && bwd_scan.lane_states && bwd_scan.fused_prefix &&
                     b * ntile <= kWideTiles;
        const size_t bwd_scan_bytes =
            size_t(scan_workspace_doubles(nrg, nblk, kPipeSections)) * sizeof(double);
        size_t aggr_f = 0;
        take(aggr_f, host_power ? bwd_scan_bytes : 0);
        fwd_bytes = off;

        off = 0;
        take(gbark, size_t(rows) * frames * nb * sizeof(float));
        take(grpart, size_t(batch) * ntile * nb * sizeof(double));
        take(gp, size_t(nrg) * len * sizeof(float));
        take(spart, size_t(nrg) * nhop * sizeof(double));
        take(aggr_b, host_power ? 0 : bwd_scan_bytes);
        take(gradtot, totals ? size_t(batch) * nb * sizeof(double) : 0);
        bwd_bytes = off;
        if (host_power) aggr_b = aggr_f;  // an offset into the forward workspace
    }

    // Regions of the stand-alone perceptual chain over given Bark spectra:
    // only the chain state (forward) and the band partials (backward).
    void build_chain(int64_t b, int64_t nframes, int nbands) {
        *this = PipeLayout();
        nb = nbands;
        batch = b;
        rows = 2 * b;
        frames = nframes;
        ntile = cdiv(frames, kTile);
        nwin = frames >= kWin ? (frames - kWin) / kStride + 1 : 0;
        size_t off = 0;
        auto take = [&](size_t &field, size_t bytes) {
            field = off;
            off = align(off + bytes);
        };
        take(keep, size_t(batch) * frames * sizeof(float));
        take(bandref, size_t(batch) * ntile * nb * sizeof(double));
        take(banddeg, size_t(batch) * ntile * nb * sizeof(double));
        take(frame, size_t(kFrameArrays) * batch * frames * sizeof(double));
        take(band, size_t(kBandArrays) * batch * nb * sizeof(double));
        take(psqm, size_t(2) * batch * nwin * sizeof(double));
        take(dist, size_t(batch) * 2 * sizeof(double));
        loud_store = 1;
        take(loud, kChainTermBytes * batch * frames * nb);
        fwd_bytes = off;
        off = 0;
        take(grpart, size_t(batch) * ntile * nb * sizeof(double));
        bwd_bytes = off;
    }

    bool region(const char *name, size_t *offset, size_t *bytes) const {
        struct Entry {
            const char *name;
            size_t off, end;
        };
        const Entry table[] = {
            {"aggr", aggr, energy},     {"energy", energy, p},
            {"p", p, f},                {"f", f, rowconst},         {"rowconst", rowconst, bark},
            {"bark", bark, keep},       {"keep", keep, bandref},    {"bandref", bandref, banddeg},
            {"banddeg", banddeg, frame}, {"frame", frame, band},    {"band", band, psqm},
            {"psqm", psqm, dist},       {"dist", dist, loud},       {"loud", loud, fwd_bytes},
        };
        for (const Entry &e : table) {
            if (std::strcmp(e.name, name) == 0) {
                *offset = e.off;
                *bytes = e.end - e.off;
                return true;
            }
        }
        return false;
    }
};

}  // namespace pesq
