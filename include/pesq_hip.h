/*
 * pesq_hip.h -- C ABI of the MI355X (gfx950) PESQ loss library.
 *
 * Every entry point takes device pointers to contiguous row-major float32
 * arrays, int64 sizes, a device pointer to a constant table built by one of
 * the *_pack functions, caller-owned workspace (size from the matching
 * *_workspace query) and an explicit hipStream_t.  Entry points enqueue work on
 * that stream and return; they never allocate, synchronise or read device
 * memory on the host, so they can be captured into a HIP graph.  Reductions
 * use a fixed order and no atomics: results are bitwise reproducible.
 *
 * Return value: PESQ_OK (0) or an error code; pesq_last_error() describes the
 * last failure of the calling thread.
 *
 * Each function replaces the reference operator named in its comment
 * (paths relative to the LarocheC/triton-pesq source tree).
 */
#ifndef PESQ_HIP_H
#define PESQ_HIP_H

#include <hip/hip_runtime_api.h>
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define PESQ_OK 0
#define PESQ_ERR_ARGUMENT 1
#define PESQ_ERR_HIP 2
#define PESQ_ERR_UNSUPPORTED 3

#define PESQ_IIR_MAX_SECTIONS 8
#define PESQ_IIR_MAX_CASCADE 32 /* biquads of a cascade (order <= 64) */
#define PESQ_NBARKS 49
#define PESQ_NFFT 512

/* bit flags of the pipeline's grad_mask */
#define PESQ_GRAD_REF 1
#define PESQ_GRAD_DEG 2

/* ----------------------------------------------------------------------- */
/* library                                                                  */
/* ----------------------------------------------------------------------- */

/* Version of this ABI (incremented on any signature or layout change). */
int pesq_abi_version(void);

/* Message of the last error on the calling thread ("" if none). */
const char *pesq_last_error(void);

/* ----------------------------------------------------------------------- */
/* constant tables (host side, no GPU call)                                 */
/* ----------------------------------------------------------------------- */

/* A causal IIR filter in parallel form: y = c0 x + sum_k s_k(x), section k a
 * direct form II transposed biquad (b0[k] + b1[k] z^-1 + b2[k] z^-2) /
 * (1 + a1[k] z^-1 + a2[k] z^-2) with zero initial state.  Packing rewrites a
 * section with b2[k] != 0 as the direct term b2[k] / a2[k] plus a section
 * without z^-2 in the numerator (the same transfer function); b2[k] != 0
 * with a2[k] == 0 is rejected. */
typedef struct pesq_iir_sections {
    int32_t count; /* 1 .. PESQ_IIR_MAX_SECTIONS */
    int32_t reserved;
    double c0;
    double b0[PESQ_IIR_MAX_SECTIONS];
    double b1[PESQ_IIR_MAX_SECTIONS];
    double b2[PESQ_IIR_MAX_SECTIONS];
    double a1[PESQ_IIR_MAX_SECTIONS];
    double a2[PESQ_IIR_MAX_SECTIONS];
} pesq_iir_sections;

/* Size in bytes of a packed IIR table. */
size_t pesq_iir_table_bytes(void);

/* Pack one filter into `out` (host memory, pesq_iir_table_bytes() bytes),
 * including the chunk transfer powers of the scan.  Replaces the host side
 * design of TritonIIR: torch_pesq/triton_ops/iir.py:520-667 (_state_space,
 * _tables). */
int pesq_iir_table_pack(const pesq_iir_sections *filter, void *out);

/* Pack a cascade (series) of `sections` full biquads into `out` (host
 * memory, sections * pesq_iir_table_bytes() bytes), one table per section.
 * `sos` is [sections][6] row major, each row (b0, b1, b2, a0, a1, a2) of
 * (b0 + b1 z^-1 + b2 z^-2) / (a0 + a1 z^-1 + a2 z^-2) as scipy.signal.tf2sos
 * returns it; 1 <= sections <= PESQ_IIR_MAX_CASCADE, a0 != 0.  The cascade
 * realisation of TritonIIR's _state_space (torch_pesq/triton_ops/iir.py:187-273
 * _cascade, :599-666), for filters whose parallel form is not accurate
 * (repeated or clustered poles, numerators longer than the denominator). */
int pesq_iir_cascade_pack(const double *sos, int sections, void *out);

/* Constants of the PESQ model (PesqLoss.__init__, torch_pesq/loss.py:61-108;
 * BarkScale, torch_pesq/bark.py:131-173; Loudness, torch_pesq/loudness.py:44-55). */
typedef struct pesq_model_constants {
    pesq_iir_sections power_filter; /* level alignment band pass, loss.py:96-99 */
    pesq_iir_sections pre_filter;   /* pre-emphasis, loss.py:102-108 */
    float window[PESQ_NFFT];        /* analysis window (n_fft taps, centred) */
    int32_t band_start[PESQ_NBARKS];/* Bark band i covers bins [start, end) */
    int32_t band_end[PESQ_NBARKS];
    double corr[PESQ_NBARKS];       /* pow_dens_correction */
    double threshs[PESQ_NBARKS];    /* hearing thresholds */
    double exps[PESQ_NBARKS];       /* Zwicker exponents */
    double width[PESQ_NBARKS];      /* width_bark */
    double total_width;             /* width_bark[1:].sum() */
    double sl;                      /* loudness constant (0.1866055) */
    int32_t nbarks;                 /* must be 49 */
    int32_t n_fft;                  /* must be 512 */
    int32_t hop;                    /* must be 256 */
    int32_t reserved;
} pesq_model_constants;

/* Size in bytes of a packed model table. */
size_t pesq_model_table_bytes(void);

/* Pack the model constants into `out` (host memory, pesq_model_table_bytes()).
 * Replaces the buffers registered by PesqLossTriton.__init__
 * (torch_pesq/triton_ops/loss.py:60-92), TritonStftBark.__init__
 * (spectral.py:634-734) and TritonPesqChain.__init__ (chain.py:1057-1078).
 * The pipeline's scans start each 1024-sample block from the two blocks
 * before it, so every filter section's state must decay below 1e-20 of
 * itself over 2048 samples (largest entry of A^2048); tables whose filters
 * decay more slowly are refused with PESQ_ERR_ARGUMENT. */
int pesq_model_table_pack(const pesq_model_constants *constants, void *out);

/* ----------------------------------------------------------------------- */
/* fused pipeline: PesqLossTriton.raw / mos / forward and their backward    */
/* ----------------------------------------------------------------------- */

/* Workspace of the forward pass.  It holds the state the backward reads and
 * must stay untouched between pesq_pipeline_forward and
 * pesq_pipeline_backward.  `len` is the 16 kHz row length. */
int pesq_pipeline_forward_workspace(int64_t batch, int64_t len, int grad_mask, size_t *bytes);

/* Scratch of the backward pass (free after the call has run). */
int pesq_pipeline_backward_workspace(int64_t batch, int64_t len, int grad_mask, size_t *bytes);

/* Distances, MOS and loss of `batch` pairs of 16 kHz signals [batch, len].
 * Replaces PesqLossTriton.raw / mos / forward
 * (torch_pesq/triton_ops/loss.py:104-147,203-215): peak normalisation,
 * level alignment, pre-emphasis, STFT, Bark, perceptual chain and the MOS
 * epilogue, in six kernels.  The
 * peak normalisation cancels in the level alignment and is not formed; the
 * workspace's "p" and "f" hold the pre-emphasised and band-passed signals in
 * the units of the input.  grad_mask (PESQ_GRAD_*) selects which inputs
 * the backward will need; it must match the backward call.  Requires
 * len >= 15 and at least 20 frames (1 + (len + len % 256 - 512) / 256).
 * batch == 0 is a no-op (no pointer is read), as is the backward's. */
int pesq_pipeline_forward(const float *ref, const float *deg, int64_t batch, int64_t len,
                          const void *model_table, double factor, int grad_mask,
                          float *d_symm, float *d_asymm, float *mos, float *loss,
                          void *fwd_workspace, hipStream_t stream);

/* Gradients w.r.t. ref and/or deg given the upstream gradients of any of the
 * four outputs (NULL = zero).  g_ref / g_deg may be NULL when not requested
 * by grad_mask.  Replaces the chain of backward kernels run by autograd
 * through PesqLossTriton (torch_pesq/triton_ops/chain.py:780-1021,
 * spectral.py:535-581, elementwise.py:233-269,607-652, iir.py:1248-1258). */
int pesq_pipeline_backward(const float *g_symm, const float *g_asymm, const float *g_mos,
                           const float *g_loss, int64_t batch, int64_t len,
                           const void *model_table, double factor, int grad_mask,
                           float *g_ref, float *g_deg, const void *fwd_workspace,
                           void *bwd_workspace, hipStream_t stream);

/* The same two passes restricted to a subset of their kernels, for per stage
 * timing.  Forward bits: 1 scan aggregates, 2 scan outputs, 4 STFT/Bark,
 * 8 chain, 16 overlapping sums + epilogue.  Backward bits: 1 chain, 2 STFT,
 * 4 adjoint scan aggregates, 8 adjoint scan outputs.  A stage reads what the
 * earlier stages wrote into the workspaces, so run the full pass first.  No
 * counterpart in the reference (its stages are separate launches). */
int pesq_pipeline_forward_stages(const float *ref, const float *deg, int64_t batch, int64_t len,
                                 const void *model_table, double factor, int grad_mask,
                                 float *d_symm, float *d_asymm, float *mos, float *loss,
                                 void *fwd_workspace, unsigned stages, hipStream_t stream);
int pesq_pipeline_backward_stages(const float *g_symm, const float *g_asymm, const float *g_mos,
                                  const float *g_loss, int64_t batch, int64_t len,
                                  const void *model_table, double factor, int grad_mask,
                                  float *g_ref, float *g_deg, const void *fwd_workspace,
                                  void *bwd_workspace, unsigned stages, hipStream_t stream);

/* Byte offset and size of a named region of the forward workspace ("p",
 * "f", "bark", "rowconst", ...), for inspection by tests.  Returns
 * PESQ_ERR_ARGUMENT for an unknown name. */
int pesq_pipeline_region(int64_t batch, int64_t len, int grad_mask, const char *name,
                         size_t *offset, size_t *bytes);

/* Names of the kernels that pesq_pipeline_forward (backward == 0) or
 * pesq_pipeline_backward (backward != 0) launches for this shape, in launch
 * order, separated by ';' (for example "iir_aggregate_kernel<5, 1,
 * PipeFwdMode, true>;...;chain_final_kernel").  Writes at most `capacity`
 * bytes including the terminating NUL into `names` (may be NULL) and the
 * full size including the NUL into *needed (may be NULL).  Host only, no GPU
 * call.  The kernel variants are chosen by grid size (lane states stored or
 * recomputed, block prefix fused or launched, frames per wavefront), so tests
 * use this to show which variants a shape exercises.  No counterpart in the
 * reference, whose Triton kernels are autotuned rather than chosen by
 * shape. */
int pesq_pipeline_kernels(int64_t batch, int64_t len, int grad_mask, int backward, char *names,
                          size_t capacity, size_t *needed);

/* Size of the static device array that serves as the workspace of
 * pesq_pipeline_forward_noalloc (32 MiB, held by each GPU the library runs on
 * until the process ends). */
#define PESQ_NOALLOC_SCRATCH_BYTES ((size_t)32 << 20)

/* pesq_pipeline_forward with grad_mask 0 (distances, MOS and loss, no
 * backward) that allocates nothing: its workspace is the library's static
 * device array of PESQ_NOALLOC_SCRATCH_BYTES on the stream's device, so the
 * caller passes only inputs and outputs.  Shapes whose forward workspace
 * (pesq_pipeline_forward_workspace with grad_mask 0) exceeds that size are
 * rejected with PESQ_ERR_ARGUMENT (about 1.5 M samples of batch x len:
 * 8 x 8 s at 16 kHz needs 21.7 MiB and fits, 16 x 8 s does not).  Calls that overlap on one GPU share the array and
 * race; calls ordered on one stream do not.  Results are bitwise those of
 * pesq_pipeline_forward.  No counterpart in the reference: this is for
 * callers that cannot allocate (code under HIP graph capture, serving loops,
 * harnesses that forbid hipMalloc). */
int pesq_pipeline_forward_noalloc(const float *ref, const float *deg, int64_t batch, int64_t len,
                                  const void *model_table, double factor, float *d_symm,
                                  float *d_asymm, float *mos, float *loss, hipStream_t stream);

/* ----------------------------------------------------------------------- */
/* IIR filter (TritonIIR, torch_pesq/triton_ops/iir.py:1266-1482)           */
/* ----------------------------------------------------------------------- */

int pesq_iir_workspace(int64_t rows, int64_t len, size_t *bytes);

/* y = lfilter(x) along rows, zero initial state; reverse != 0 applies the
 * time reversed filter, the adjoint (iir.py:1232-1258).  `sections` is the
 * count of the packed filter (pesq_iir_sections.count). */
int pesq_iir_apply(const float *x, float *y, int64_t rows, int64_t len, const void *iir_table,
                   int sections, int reverse, void *workspace, hipStream_t stream);

/* Workspace of pesq_iir_cascade_apply: the scan workspace plus up to two
 * float64 [rows, len] intermediate signals. */
int pesq_iir_cascade_workspace(int64_t rows, int64_t len, int sections, size_t *bytes);

/* y = lfilter(x) through a packed cascade of `sections` biquads (TritonIIR
 * forward / _IIRFunction, iir.py:1232-1258,1451-1482): one scan pass per
 * section with float64 state, float64 signals between the passes; reverse
 * != 0 applies the adjoint (every pass time reversed). */
int pesq_iir_cascade_apply(const float *x, float *y, int64_t rows, int64_t len,
                           const void *cascade_tables, int sections, int reverse,
                           void *workspace, hipStream_t stream);

/* ----------------------------------------------------------------------- */
/* resampler (TritonResample, torch_pesq/triton_ops/resample.py:442-574)    */
/* ----------------------------------------------------------------------- */

/* y[l new_step + j] = sum_k kernel[j, k] x[l orig_step + k - width] for the
 * non-zero taps tap_lo[j] <= k < tap_hi[j] of each phase ([new_step] int32
 * each); kernel is [new_step, width_total] float32, width_total =
 * 2 width + orig_step; x reads as zero outside [0, n_in).  Replaces
 * _resample_fwd_kernel (resample.py:113-175). */
int pesq_resample_forward(const float *x, float *y, int64_t rows, int64_t n_in, int64_t n_out,
                          const float *kernel, const int32_t *tap_lo, const int32_t *tap_hi,
                          int64_t orig_step, int64_t new_step, int64_t width,
                          int64_t width_total, hipStream_t stream);

/* Adjoint of pesq_resample_forward, a gather over input samples; phase_lo /
 * phase_hi ([width_total] int32) bound the phases with a non-zero tap k.
 * Replaces _resample_bwd_kernel (resample.py:178-243). */
int pesq_resample_backward(const float *grad_y, float *grad_x, int64_t rows, int64_t n_in,
                           int64_t n_out, const float *kernel, const int32_t *phase_lo,
                           const int32_t *phase_hi, int64_t orig_step, int64_t new_step,
                           int64_t width, int64_t width_total, hipStream_t stream);

/* Tiled resampler.  pesq_resample_plan turns the filter bank (host memory,
 * [new_step, width_total] float32, with the non-zero tap range of each phase)
 * into compact zero-padded tap tables for a forward and an adjoint kernel
 * that stage each workgroup's samples in LDS: it fills `info` and, when
 * `plan` is not NULL, writes info->bytes bytes of tables (host memory, to be
 * copied to the device).  fwd_span / bwd_span of 0 mean the rate pair's
 * window is too wide for the LDS tile; the untiled entry points above then
 * apply.  The forward sums the same terms in the same order as
 * pesq_resample_forward.  The adjoint of a rate pair with new_step > 1 is
 * itself a resampler from the new rate to the old one (upsampling by
 * orig_step and downsampling by new_step, with the bank transposed): input i
 * receives the contiguous run of outputs whose taps cover it, adj_taps of
 * them at most, so the plan holds that transposed bank (adj_*) and the
 * adjoint runs the forward's tiled kernel on it, summing over the outputs in
 * ascending order (the untiled adjoint adds the same terms sweep by sweep).
 * Replaces _resample_fwd_kernel / _resample_bwd_kernel (resample.py:113-243). */
typedef struct pesq_resample_plan_info {
    int32_t orig_step, new_step, width, width_total;
    int32_t taps;             /* longest non-zero tap run of one phase */
    int32_t off_min, off_max; /* extremes of tap_lo[j] - width */
    int32_t phases;           /* most phases reading one tap column */
    int32_t sweeps;           /* ceil(width_total / orig_step) */
    int32_t columns;          /* sweeps * orig_step */
    int32_t fwd_span, bwd_span; /* floats staged per workgroup, 0 = not tiled */
    int64_t bytes;            /* size of the plan tables */
    int64_t off_offs, off_cols, off_col_lo, off_taps64, off_row64; /* table offsets */
    /* the adjoint as a resampler from new_step to orig_step (new_step > 1):
     * gx[l orig + j] = sum_{t < adj_taps} adj[t][j] gy[l new_step + adj_offs[j] + t] */
    int32_t adj_taps, adj_off_min, adj_off_max, adj_span; /* adj_span 0: not used */
    int64_t off_adj_taps, off_adj_offs;                   /* table offsets */
} pesq_resample_plan_info;

int pesq_resample_plan(const float *kernel, const int32_t *tap_lo, const int32_t *tap_hi,
                       int64_t orig_step, int64_t new_step, int64_t width, int64_t width_total,
                       pesq_resample_plan_info *info, void *plan);

int pesq_resample_plan_forward(const float *x, float *y, int64_t rows, int64_t n_in,
                               int64_t n_out, const pesq_resample_plan_info *info,
                               const void *plan, hipStream_t stream);

int pesq_resample_plan_backward(const float *grad_y, float *grad_x, int64_t rows, int64_t n_in,
                                int64_t n_out, const pesq_resample_plan_info *info,
                                const void *plan, hipStream_t stream);

/* The two calls above for two signals of one shape at once (x0 -> y0 and
 * x1 -> y1, each [rows, n]), in one launch over 2 rows: the same outputs as
 * two single calls, bit for bit, without stacking the signals into one
 * tensor first.  Replaces the resampling of the stacked reference and
 * degraded batch in PesqLossTriton.raw (triton_ops/loss.py:130-136) and its
 * adjoint. */
int pesq_resample_plan_forward_pair(const float *x0, float *y0, const float *x1, float *y1,
                                    int64_t rows, int64_t n_in, int64_t n_out,
                                    const pesq_resample_plan_info *info, const void *plan,
                                    hipStream_t stream);

int pesq_resample_plan_backward_pair(const float *grad_y0, float *grad_x0, const float *grad_y1,
                                     float *grad_x1, int64_t rows, int64_t n_in, int64_t n_out,
                                     const pesq_resample_plan_info *info, const void *plan,
                                     hipStream_t stream);

/* ----------------------------------------------------------------------- */
/* STFT / Bark (TritonStftBark, torch_pesq/triton_ops/spectral.py:584-774)  */
/* ----------------------------------------------------------------------- */

/* bark[r, t, i] = corr_i sum_{f in band i} |DFT(window . x[r, 256 t : 256 t + 512])_f|^2
 * for t < 1 + (n_padded - 512) / 256, samples at or beyond len read as zero,
 * DC dropped.  model_table from pesq_model_table_pack (filters may be absent).
 * Replaces _fwd_kernel (spectral.py:229-332). */
int pesq_stft_bark_forward(const float *x, int64_t rows, int64_t len, int64_t n_padded,
                           const void *model_table, float *bark, hipStream_t stream);

/* Vector-Jacobian product of pesq_stft_bark_forward: g_x [rows, len].
 * Replaces _bwd_frame_kernel + _bwd_gather_kernel (spectral.py:334-440). */
int pesq_stft_bark_backward(const float *g_bark, const float *x, int64_t rows, int64_t len,
                            int64_t n_padded, const void *model_table, float *g_x,
                            hipStream_t stream);

/* General geometry (TritonStftBark with any n_fft / hop_length / filterbank,
 * spectral.py:584-774): n_fft a power of two in [32, 1024], hop >= 1, 1..128
 * bands.  Frames t < 1 + (n_padded - n_fft) / hop start at t * hop. */

/* Size in bytes of a packed general STFT table. */
size_t pesq_stft_table_bytes(void);

/* Pack the general STFT constants into `out` (host memory,
 * pesq_stft_table_bytes() bytes): window [n_fft] (already centred), bands
 * [band_start[i], band_end[i]) over bins 0 .. n_fft / 2 - 1 (sorted, disjoint),
 * corr [nbarks].  Replaces bark_segments / _twiddles (spectral.py:138-224). */
int pesq_stft_table_pack(int n_fft, int hop, const float *window, int nbarks,
                         const int32_t *band_start, const int32_t *band_end,
                         const double *corr, void *out);

/* Scratch of pesq_stft_backward: [rows, frames, n_fft] float32. */
int pesq_stft_workspace(int64_t rows, int64_t len, int64_t n_padded, int n_fft, int hop,
                        size_t *bytes);

/* bark [rows, frames, nbarks] of x [rows, len] (zero beyond len), as
 * pesq_stft_bark_forward for the general geometry (_fwd_kernel,
 * spectral.py:229-332). */
int pesq_stft_forward(const float *x, int64_t rows, int64_t len, int64_t n_padded,
                      const void *stft_table, int n_fft, int hop, int nbarks, float *bark,
                      hipStream_t stream);

/* g_x [rows, len] from g_bark, the vector-Jacobian product of
 * pesq_stft_forward (_bwd_frame_kernel + _bwd_gather_kernel,
 * spectral.py:334-440); samples no frame covers get zero. */
int pesq_stft_backward(const float *g_bark, const float *x, int64_t rows, int64_t len,
                       int64_t n_padded, const void *stft_table, int n_fft, int hop,
                       int nbarks, float *g_x, void *workspace, hipStream_t stream);

/* ----------------------------------------------------------------------- */
/* perceptual chain (TritonPesqChain, torch_pesq/triton_ops/chain.py:1024-1126) */
/* ----------------------------------------------------------------------- */

/* Pack the chain constants of `nbands` bands (1 .. 128) into `out` (host
 * memory, pesq_model_table_bytes() bytes): hearing thresholds (> 0), loudness
 * exponents, band widths in Bark, their total over bands 1.. and sl.  The
 * constructor of TritonPesqChain (chain.py:1057-1078).  A table from
 * pesq_model_table_pack serves the 49 band chain as well. */
int pesq_chain_table_pack(int nbands, const double *threshs, const double *exps,
                          const double *widths, double total_width, double sl, void *out);

int pesq_chain_forward_workspace(int64_t batch, int64_t frames, int nbands, size_t *bytes);
int pesq_chain_backward_workspace(int64_t batch, int64_t frames, int nbands, size_t *bytes);

/* (d_symm, d_asymm)[batch] of two Bark spectrograms [batch, frames, nbands]
 * (nbands 1 .. 128, as packed in model_table); needs at least 20 frames.
 * batch == 0 is a no-op, as in the reference (test_triton_chain.py:799-806),
 * and so is the backward's.
 * Replaces the 7 forward kernels of _ChainFunction.forward (chain.py:768-940). */
int pesq_chain_forward(const float *ref_bark, const float *deg_bark, int64_t batch,
                       int64_t frames, int nbands, const void *model_table, float *d_symm,
                       float *d_asymm, void *fwd_workspace, hipStream_t stream);

/* Gradients w.r.t. both spectrograms given those of the distances (NULL =
 * zero).  Replaces _ChainFunction.backward (chain.py:942-1021). */
int pesq_chain_backward(const float *g_symm, const float *g_asymm, const float *ref_bark,
                        const float *deg_bark, int64_t batch, int64_t frames, int nbands,
                        const void *model_table, float *g_ref_bark, float *g_deg_bark,
                        const void *fwd_workspace, void *bwd_workspace, hipStream_t stream);

/* ----------------------------------------------------------------------- */
/* element-wise stages (torch_pesq/triton_ops/elementwise.py)               */
/* ----------------------------------------------------------------------- */

/* Scratch of the element-wise reductions for `rows` rows. */
int pesq_elementwise_workspace(int64_t rows, size_t *bytes);

/* peak[b] = max(max|ref[b]|, max|deg[b]|); out = x / peak (IEEE division).
 * out_ref / out_deg may point into one stacked [2 batch, len] buffer.
 * Replaces _peak_partial_kernel + _peak_apply_kernel (elementwise.py:74-133). */
int pesq_peak_normalize_forward(const float *ref, const float *deg, int64_t batch, int64_t len,
                                float *out_ref, float *out_deg, float *peak, void *workspace,
                                hipStream_t stream);

/* g / peak for the requested halves (NULL skips one); the peak is a constant.
 * Replaces _div_pair_kernel (elementwise.py:136-162). */
int pesq_peak_normalize_backward(const float *g_ref, const float *g_deg, const float *peak,
                                 int64_t batch, int64_t len, float *out_ref, float *out_deg,
                                 hipStream_t stream);

/* y = (x head) tail with head_k = (k+1)/16 (k < 15), tail_k = (len-k)/16 (last
 * 15); its own adjoint.  Replaces _edge_ramp_kernel (elementwise.py:308-331). */
int pesq_edge_ramp(const float *x, float *y, int64_t rows, int64_t len, hipStream_t stream);

/* power = sum filtered^2 / (n_flt + 5120) / 1.04684, scale = sqrt(1e7 / power),
 * out = signal * scale; state[rows, 2] (float64) = {power, scale} for the
 * backward.  Replaces _dot_partial_kernel + _align_apply_kernel
 * (elementwise.py:416-481). */
int pesq_align_scale_forward(const float *signal, const float *filtered, int64_t rows,
                             int64_t n_sig, int64_t n_flt, float *out, double *state,
                             void *workspace, hipStream_t stream);

/* g_signal = grad scale; g_filtered = 2 filtered (-0.5 S scale / power) / D
 * with S = sum grad signal (either output may be NULL).  Replaces
 * _mul_bcast_kernel + _align_grad_filtered_kernel (elementwise.py:484-536). */
int pesq_align_scale_backward(const float *grad, const float *signal, const float *filtered,
                              const double *state, int64_t rows, int64_t n_sig, int64_t n_flt,
                              float *g_signal, float *g_filtered, void *workspace,
                              hipStream_t stream);

/* mos = 0.999 + 4 / (1 + exp(-1.3669 (4.5 - 0.1 ds - 0.0309 da) + 3.8224)),
 * loss = factor (0.1 ds + 0.0309 da).  Replaces _epilogue_kernel
 * (elementwise.py:683-700). */
int pesq_epilogue_forward(const float *d_symm, const float *d_asymm, int64_t batch, double factor,
                          float *mos, float *loss, hipStream_t stream);

/* Gradients of both distances from those of MOS and/or loss (NULL = zero).
 * Replaces _epilogue_bwd_kernel (elementwise.py:703-747). */
int pesq_epilogue_backward(const float *d_symm, const float *d_asymm, const float *g_mos,
                           const float *g_loss, int64_t batch, double factor, float *g_symm,
                           float *g_asymm, hipStream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* PESQ_HIP_H */
