"""Float64 CPU oracle of the PESQ loss pipeline.

TEST INFRASTRUCTURE ONLY.  Only ``tests/``, ``__graft_entry__.smoke()`` and the
``cpu_baseline`` leg of ``bench.py`` may import this module, and only as the
checker.  The shipped package never imports, links or runs anything here.

Every stage restates the reference pipeline in float64 torch-CPU arithmetic
(autograd supplies the gradients), following:

* ``torch_pesq/loss.py:111-141``  ``align_level`` (band pass power to 1e7)
* ``torch_pesq/loss.py:144-169``  ``preemphasize`` (edge ramp + lfilter)
* ``torch_pesq/loss.py:172-268``  ``raw`` (peak, resample, pad, STFT, chain)
* ``torch_pesq/loss.py:271-322``  ``mos`` / ``forward``
* ``torch_pesq/triton_ops/reference.py:28-323`` the stage decomposition
* ``tests/test_triton_loss.py:101-150`` the float64 promotion recipe: every
  constant is the float32/float64 value the reference module holds, promoted
  to float64.
* torchaudio ``_get_sinc_resample_kernel`` / ``_apply_sinc_resample_kernel``
  (third party, absent here; restated from its published algorithm, see
  :func:`sinc_resample_kernel`).

How each part is pinned (``tests/test_oracle.py``):

* tables: equal to ``tests/golden/tables.json`` (parsed from the reference)
  and to the filterbank known answer of ``tests/test_fbank.py:5-11``;
* ``lfilter``: ``scipy.signal.lfilter`` (the difference equation) against a
  pure-Python recursion on short inputs, the second order section cascade,
  and the adjoint identity ``<y, H x> = <H^T y, x>``;
* ``stft_bark``: a direct float64 DFT on short inputs, the frame count known
  answer (4000 samples -> 14 frames, ``test_triton_spectral.py:397-412``) and
  finite differences;
* formula constants: every scalar of the formulas lives in :data:`FORMULA`,
  which must equal, name by name, the literals ``tests/golden/make_tables.py``
  parses from the reference's statements (``loss.py``, ``loudness.py``,
  ``bark.py``, ``triton_ops/reference.py``); no other numeric literal than a
  structural 0, 1 or 2 appears in the formula functions;
* chain, step by step, against closed-form consequences that a misread
  constant or a misplaced term fails (each test also plants such a mistake and
  sees it fail): the loudness law's zero at the threshold, its ``sl x^e``
  asymptote and its slope above the threshold; the dead zone's
  ``0.75 L_ref`` / ``0`` / ``-0.375 L_ref`` answers; the silence decision and
  the all-frame band means; the band and frame ratios' offsets, smoothing and
  clamps; the asymmetry factor at ``2.5^1.2`` and its cut and cap; ``h(0) =
  0.01^0.04`` (the 0.83175 of ``test_triton_chain.py:725-750``); the norms'
  absolute scale ``sqrt(W) w_k |d|`` and ``w_k |d|``; the overlapping sums of
  one non-zero frame ``v 20^(-1/6) sqrt(m / nwin)``; whole-chain distances of
  constant single-band spectra in closed form; plus the identical-input known
  answer (``1e-20 / h`` floor, ``test_triton_chain.py:365-383``), a float64
  finite difference check of the autograd gradient, and a pure-Python loop
  evaluation on a tiny spectrum;
* epilogue: values evaluated by hand from the published ITU-T P.862 raw score
  and P.862.2 wideband mapping (4.6439 at zero disturbance);
* pipeline: scale invariance (``test_triton_elementwise.py:1396-1450``),
  batch independence, ``loss(ref, ref) ~ 0`` (``test_torch.py:18-27``);
* resampler taps: width / length known answers of
  ``test_triton_resample.py:13,177-181,620-647,685-686``, unit DC gain,
  symmetry and identity at equal rates.  The exact torchaudio taps are
  **parity unpinned** (torchaudio is not installed and the reference stores
  no tap values).
"""

import json
import math
from functools import lru_cache
from pathlib import Path

import numpy as np
import torch
from scipy import interpolate
from scipy.signal import butter, lfilter as scipy_lfilter

ROOT = Path(__file__).resolve().parents[1]
TABLES = json.loads((ROOT / "tests" / "golden" / "tables.json").read_text())

#: Every scalar constant of the loss's formulas, typed from a reading of the
#: reference (the line each is read from).  ``tests/test_oracle.py`` checks
#: this dict, key by key, against the values ``tests/golden/make_tables.py``
#: parses from the reference's source text, and the functions below read
#: their constants only from here.
FORMULA = {
    # level alignment, torch_pesq/loss.py:132-139
    "align_pad": 5120,
    "align_divisor": 1.04684,
    "align_target_base": 10,
    "align_target_exponent": 7,
    # edge ramp, torch_pesq/loss.py:163-165
    "ramp_length": 15,
    "ramp_points": 16,
    "ramp_divisor": 16.0,
    # N % 256 padding, torch_pesq/loss.py:191-192
    "pad_multiple": 256,
    # silent frames and band means, loss.py:206, loudness.py:102
    "silent_threshold_factor": 100.0,
    "silent_energy": 1e7,
    "mean_threshold_factor": 100.0,
    # band power ratio, loss.py:212-216
    "band_ratio_offset": 1000,
    "band_ratio_min": 0.01,
    "band_ratio_max": 100.0,
    # frame power ratio, loss.py:220-228
    "total_threshold_factor": 1,
    "frame_ratio_offset": 5e3,
    "frame_smooth_current": 0.8,
    "frame_smooth_previous": 0.2,
    "frame_ratio_min": 3e-4,
    "frame_ratio_max": 5.0,
    # Zwicker loudness, loudness.py:124-129 and its exponents, loudness.py:52-55
    "loudness_threshold_scale": 2.0,
    "loudness_half": 0.5,
    "loudness_one": 1,
    "loudness_below_threshold": 0.0,
    "exponent_numerator": 6,
    "exponent_offset": 2.0,
    "exponent_min": 1.0,
    "exponent_max": 2.0,
    "exponent_power": 0.15,
    # disturbance and its norms, loss.py:235-249, bark.py:193-195
    "deadzone": 0.25,
    "symm_norm_p": 2,
    "asymm_norm_p": 1,
    "norm_first_band": 1,
    "distance_floor": 1e-20,
    "asymm_offset": 50.0,
    "asymm_exponent": 1.2,
    "asymm_cut": 3.0,
    "asymm_cut_value": 0.0,
    "asymm_cap": 12.0,
    # frame weighting and cap, loss.py:252-253
    "h_offset": 1e5,
    "h_scale": 1e7,
    "h_exponent": 0.04,
    "distance_cap": 45.0,
    # overlapping sums, loss.py:256-266
    "psqm_window": 20,
    "psqm_stride": 10,
    "psqm_power": 6,
    # MOS and loss, loss.py:292-295,322
    "pesq_offset": 4.5,
    "pesq_symm_weight": 0.1,
    "pesq_asymm_weight": 0.0309,
    "mos_floor": 0.999,
    "mos_span": 4,
    "mos_slope": 1.3669,
    "mos_shift": 3.8224,
    # loudness calibration passed to the chain, triton_ops/reference.py:315-322
    "sl": 0.1866055,
}
F = FORMULA
SL = F["sl"]
WINDOW, STRIDE = F["psqm_window"], F["psqm_stride"]


# ---------------------------------------------------------------------------
# constants, promoted to float64 exactly as the reference module holds them
# ---------------------------------------------------------------------------


def _interp(values, nelms_new):
    """``torch_pesq/bark.py:81-99``: scipy interp1d over the table index."""

    table = np.asarray(values, dtype=np.float64)
    curve = interpolate.interp1d(np.arange(table.shape[0]), table)
    return torch.tensor(curve(np.linspace(0, 49.0, nelms_new, endpoint=False)))


def bark_fbank(nfreqs: int = 256, nbarks: int = 49) -> torch.Tensor:
    """Binary Bark filterbank ``[nbarks, nfreqs]`` (``torch_pesq/bark.py:140-165``).

    The default geometry uses the standard's bin counts per band; any other
    one places band ``i`` at its interpolated centre with its interpolated
    width (bins of 8000 / nfreqs Hz), clipped to start after the previous band.
    """

    fbank = torch.zeros(nbarks, nfreqs, dtype=torch.float64)
    if nfreqs == 256 and nbarks == 49:
        edges = np.concatenate([[0], np.cumsum(TABLES["nr_of_hz_bands_per_bark_band_16k"])])
        for band in range(nbarks):
            fbank[band, int(edges[band]) : int(edges[band + 1])] = 1.0
        return fbank
    width_hz = _interp(TABLES["width_of_band_hz_16k"], nbarks)
    centre_hz = _interp(TABLES["centre_of_band_hz_16k"], nbarks)
    prev, bin_width = 0, 8000.0 / nfreqs
    for band in range(nbarks):
        stride = float(width_hz[band]) / bin_width
        centre = float(centre_hz[band]) / bin_width
        start = max(prev, int(math.floor(centre - stride / 2)))
        end = min(nfreqs, int(math.ceil(centre + stride / 2)))
        fbank[band, start:end] = 1.0
        prev = end
    return fbank


def stft_bark_op(signal, window, fbank, corr, n_fft: int, hop: int, n_padded: int = None):
    """The stand-alone STFT / Bark operator in float64 (``reference.py:79-127``).

    ``signal`` ``[rows, N]`` is zero padded to ``n_padded``; frames
    ``t < 1 + (n_padded - n_fft) // hop`` start at ``t hop``; ``window`` has at
    most ``n_fft`` taps and is centred like ``torch.stft`` does; DC dropped,
    bins ``0 .. n_fft / 2 - 1`` summed per band and scaled by ``corr``.
    """

    signal = signal.double()
    n_padded = signal.shape[1] if n_padded is None else n_padded
    signal = torch.nn.functional.pad(signal, (0, n_padded - signal.shape[1]))
    window = torch.as_tensor(window).double()
    spec = torch.stft(
        signal,
        n_fft=n_fft,
        hop_length=hop,
        win_length=window.shape[0],
        window=window,
        center=False,
        normalized=False,
        return_complex=True,
    )
    spec = spec.abs().pow(2).swapaxes(1, 2)
    spec = torch.cat([torch.zeros_like(spec[:, :, :1]), spec[:, :, 1:]], dim=2)
    bark = torch.matmul(spec[:, :, :-1], torch.as_tensor(fbank).double().t())
    return bark * torch.as_tensor(corr).double().reshape(-1)


@lru_cache(maxsize=None)
def constants(nbarks: int = 49, n_fft: int = 512):
    """All constants of the pipeline as float64 tensors.

    * ``power_b/power_a``: ``butter(5, [325, 3250], fs=16000, 'band')`` stored
      as a float32 Parameter (``loss.py:96-99``), promoted to float64;
    * ``pre_b/pre_a``: the float32 pre-emphasis Parameter (``loss.py:102-108``);
    * ``window``: ``torch.hann_window(win_length)`` (float32, periodic,
      ``loss.py:79-87``);
    * Bark tables (``bark.py:134-173``), thresholds and exponents
      (``loudness.py:44-55``; the exponents are float32 values).
    """

    assert n_fft == 512 and nbarks == 49, "the oracle covers the default PESQ setup"

    nfreqs = n_fft // 2
    counts = TABLES["nr_of_hz_bands_per_bark_band_16k"]
    edges = np.concatenate([[0], np.cumsum(counts)])
    fbank = torch.zeros(nbarks, nfreqs, dtype=torch.float64)
    for band in range(nbarks):
        fbank[band, int(edges[band]) : int(edges[band + 1])] = 1.0

    width_bark = _interp(TABLES["width_of_band_bark_16k"], nbarks)
    corr = _interp(TABLES["pow_dens_correction_factor_16k"], nbarks) * TABLES["Sp_16k"]
    threshs = _interp(TABLES["abs_thresh_power_16k"], nbarks)

    exp32 = F["exponent_numerator"] / (
        torch.tensor(TABLES["centre_of_band_bark_16k"], dtype=torch.float32) + F["exponent_offset"]
    )
    exp32 = exp32.clamp(min=F["exponent_min"], max=F["exponent_max"]) ** F["exponent_power"]
    exp32 = exp32 * TABLES["zwicker_power"]

    design = TABLES["power_filter_design"]
    pb, pa = butter(design["order"], design["band_hz"], fs=design["fs"], btype="band")
    power = torch.as_tensor(np.stack([pb, pa]), dtype=torch.float32).double()
    pre = torch.tensor(
        [TABLES["pre_filter_b"], TABLES["pre_filter_a"]], dtype=torch.float32
    ).double()

    return {
        "fbank": fbank,
        "corr": corr,
        "width_bark": width_bark,
        "total_width": width_bark[1:].sum(),
        "threshs": threshs,
        "exp": exp32.double(),
        "window": torch.hann_window(n_fft).double(),
        "power_b": power[0],
        "power_a": power[1],
        "pre_b": pre[0],
        "pre_a": pre[1],
        "n_fft": n_fft,
        "hop": 256,
    }


# ---------------------------------------------------------------------------
# lfilter in float64 with its adjoint
# ---------------------------------------------------------------------------


def lfilter64(x: np.ndarray, b, a, reverse: bool = False) -> np.ndarray:
    """Zero state difference equation along the last axis, float64.

    ``reverse`` filters the time reversed signal and reverses the result, the
    vector-Jacobian product of the causal filter.
    """

    b = np.asarray(b, dtype=np.float64)
    a = np.asarray(a, dtype=np.float64)
    x = np.asarray(x, dtype=np.float64)
    if reverse:
        # .copy() also normalises the strides of length-1 axes
        return scipy_lfilter(b, a, x[..., ::-1], axis=-1)[..., ::-1].copy()
    return scipy_lfilter(b, a, x, axis=-1).copy()


class _LFilter(torch.autograd.Function):
    @staticmethod
    def forward(ctx, x, b, a):
        ctx.coeffs = (b.detach().cpu().numpy(), a.detach().cpu().numpy())
        out = lfilter64(x.detach().cpu().numpy(), *ctx.coeffs)
        return torch.from_numpy(out).to(x.dtype)

    @staticmethod
    def backward(ctx, grad):
        out = lfilter64(grad.detach().cpu().numpy(), *ctx.coeffs, reverse=True)
        return torch.from_numpy(out).to(grad.dtype), None, None


def lfilter(x: torch.Tensor, b: torch.Tensor, a: torch.Tensor) -> torch.Tensor:
    """Differentiable float64 ``lfilter(x, a, b, clamp=False)``."""

    return _LFilter.apply(x.double(), b.double(), a.double())


# ---------------------------------------------------------------------------
# resampler (torchaudio published algorithm, restated)
# ---------------------------------------------------------------------------


def sinc_resample_kernel(
    orig_freq: int,
    new_freq: int,
    lowpass_filter_width: int = 6,
    rolloff: float = 0.99,
    resampling_method: str = "sinc_interp_hann",
    beta=None,
):
    """Windowed sinc filter bank ``[new_step, width_total]`` and the pad width.

    Restates torchaudio's ``_get_sinc_resample_kernel`` (called by the
    reference at ``triton_ops/resample.py:512-521`` and, through
    ``torchaudio.transforms.Resample``, at ``loss.py:76``).  With the rates
    reduced by their gcd, ``base = min(orig, new) * rolloff``,
    ``width = ceil(lpw * orig / base)``, and for output phase ``j`` and tap
    ``k``: ``t = (-j / new + (k - width) / orig) * base`` clamped to
    ``[-lpw, lpw]``; the taps are ``sinc(pi t) * window(t) * base / orig`` with
    the Hann window ``cos(pi t / (2 lpw))**2`` (or the Kaiser window).  The
    phase term ``-j / new`` is formed in float32 (torchaudio divides an integer
    ``arange`` by ``new``), everything else in float64, and the bank is
    returned in float32.
    """

    if resampling_method not in ("sinc_interp_hann", "sinc_interp_kaiser"):
        raise ValueError(f"Invalid resampling method: {resampling_method}")
    if lowpass_filter_width <= 0:
        raise ValueError("Low pass filter width should be positive.")

    gcd = math.gcd(int(orig_freq), int(new_freq))
    orig, new = int(orig_freq) // gcd, int(new_freq) // gcd

    base = min(orig, new) * rolloff
    width = math.ceil(lowpass_filter_width * orig / base)

    idx = torch.arange(-width, width + orig, dtype=torch.float64)[None, None] / orig
    phase = torch.arange(0, -new, -1)[:, None, None] / new  # float32
    t = (phase + idx) * base
    t = t.clamp(-lowpass_filter_width, lowpass_filter_width)

    if resampling_method == "sinc_interp_hann":
        window = torch.cos(t * math.pi / lowpass_filter_width / 2) ** 2
    else:
        beta = 14.769656459379492 if beta is None else beta
        beta_t = torch.tensor(float(beta))
        window = torch.i0(beta_t * torch.sqrt(1 - (t / lowpass_filter_width) ** 2)) / torch.i0(beta_t)

    t = t * math.pi
    kernels = torch.where(t == 0, torch.tensor(1.0, dtype=t.dtype), t.sin() / t)
    kernels = kernels * window * (base / orig)

    return kernels.to(torch.float32).reshape(new, -1), width


def resample_length(n_samples: int, orig_freq: int, new_freq: int) -> int:
    """torchaudio's output length: ``ceil`` of ``new * n / orig`` in float32."""

    gcd = math.gcd(int(orig_freq), int(new_freq))
    orig, new = int(orig_freq) // gcd, int(new_freq) // gcd
    return int(torch.ceil(torch.as_tensor(new * n_samples / orig, dtype=torch.float32)).long())


def resample(x: torch.Tensor, orig_freq: int, new_freq: int = 16000, **kwargs) -> torch.Tensor:
    """Polyphase sinc resampling in float64 (torchaudio's conv form).

    ``y = conv1d(pad(x, (width, width + orig)), K, stride=orig)``, phases
    interleaved and cut to :func:`resample_length`.
    """

    if orig_freq == new_freq:
        return x

    kernel, width = sinc_resample_kernel(orig_freq, new_freq, **kwargs)
    gcd = math.gcd(int(orig_freq), int(new_freq))
    orig = int(orig_freq) // gcd

    rows, n = x.shape
    padded = torch.nn.functional.pad(x.double(), (width, width + orig))
    out = torch.nn.functional.conv1d(padded[:, None], kernel.double()[:, None, :], stride=orig)
    out = out.transpose(1, 2).reshape(rows, -1)
    return out[:, : resample_length(n, orig_freq, new_freq)]


# ---------------------------------------------------------------------------
# pipeline stages
# ---------------------------------------------------------------------------


def peak_normalize(ref: torch.Tensor, deg: torch.Tensor):
    """Common peak ``max(max|ref|, max|deg|)`` per item (``loss.py:179-183``)."""

    peak = torch.max(deg.abs().amax(1, keepdim=True), ref.abs().amax(1, keepdim=True))
    return ref / peak, deg / peak, peak


def align_level(signal: torch.Tensor, c=None) -> torch.Tensor:
    """``loss.py:127-139`` / ``reference.py:28-51``."""

    c = constants() if c is None else c
    filtered = lfilter(signal, c["power_b"], c["power_a"])
    power = (filtered**2).sum(dim=1, keepdim=True) / (filtered.shape[1] + F["align_pad"])
    power = power / F["align_divisor"]
    target = F["align_target_base"] ** F["align_target_exponent"]
    return signal * (target / power).sqrt()


def edge_ramp(signal: torch.Tensor) -> torch.Tensor:
    """First and last 15 samples times ``k/16``, applied in that order (``loss.py:163-165``)."""

    n = F["ramp_length"]
    emp = torch.linspace(0, n, F["ramp_points"], dtype=torch.float32)[1:] / F["ramp_divisor"]
    emp = emp.to(signal.dtype)
    out = signal.clone()
    out[:, :n] = out[:, :n] * emp
    out[:, -n:] = out[:, -n:] * torch.flip(emp, dims=(0,))
    return out


def preemphasize(signal: torch.Tensor, c=None) -> torch.Tensor:
    """``loss.py:163-167`` / ``reference.py:54-76``."""

    c = constants() if c is None else c
    return lfilter(edge_ramp(signal), c["pre_b"], c["pre_a"])


def n_frames(n_samples: int, n_fft: int = 512, hop: int = 256) -> int:
    """Frames after the reference's ``length % 256`` padding (``loss.py:191-192``)."""

    padded = n_samples + n_samples % F["pad_multiple"]
    return 1 + (padded - n_fft) // hop


def stft_bark(signal: torch.Tensor, c=None) -> torch.Tensor:
    """Pad by ``N % 256``, float64 STFT, DC dropped, Bark sums (``reference.py:79-127``)."""

    c = constants() if c is None else c
    signal = torch.nn.functional.pad(signal, (0, signal.shape[1] % F["pad_multiple"]))
    spec = torch.stft(
        signal,
        n_fft=c["n_fft"],
        hop_length=c["hop"],
        win_length=c["window"].shape[0],
        window=c["window"].to(signal.dtype),
        center=False,
        normalized=False,
        return_complex=True,
    )
    spec = spec.abs().pow(2).swapaxes(1, 2)
    spec = torch.cat([torch.zeros_like(spec[:, :, :1]), spec[:, :, 1:]], dim=2)
    bark = torch.matmul(spec[:, :, :-1], c["fbank"].t().to(spec.dtype))
    return bark * c["corr"].to(spec.dtype)


def total_audible(spec, threshs, factor):
    """Energy of the bands above ``factor`` times their threshold, per frame
    (``loudness.py:61-79``)."""

    return (spec * (spec > threshs * factor)).sum(dim=2)


def silent_frames(ref, threshs):
    """Frames whose reference energy above ``100 th`` is below ``1e7``
    (``loss.py:205-206``)."""

    return total_audible(ref, threshs, F["silent_threshold_factor"]) < F["silent_energy"]


def band_means(spec, threshs, silent):
    """Per band mean over *all* frames of the powers above ``100 th`` in the
    non-silent frames (``loudness.py:82-105``)."""

    mask = (spec > threshs * F["mean_threshold_factor"]) * (~silent.unsqueeze(2))
    return (spec * mask).mean(dim=1)


def band_ratio(mean_ref, mean_deg):
    """``clamp((m_deg + 1000) / (m_ref + 1000), 0.01, 100)`` per band (``loss.py:212-216``)."""

    off = F["band_ratio_offset"]
    return ((mean_deg + off) / (mean_ref + off)).clamp(min=F["band_ratio_min"], max=F["band_ratio_max"])


def frame_ratio(taer, tad):
    """Frame power ratio ``(taer + 5e3) / (tad + 5e3)``, smoothed
    ``0.8 f_t + 0.2 f_(t-1)`` for ``t > 0`` and clamped to ``[3e-4, 5]``
    (``loss.py:219-228``)."""

    off = F["frame_ratio_offset"]
    f = (taer + off) / (tad + off)
    smoothed = f[:, 1:] * F["frame_smooth_current"] + f[:, :-1] * F["frame_smooth_previous"]
    f = torch.cat([f[:, :1], smoothed], dim=1)
    return f.clamp(min=F["frame_ratio_min"], max=F["frame_ratio_max"])


def loudness(pow_dens, threshs, exp, sl):
    """Zwicker loudness ``sl (2 th)^e ((0.5 + 0.5 x / th)^e - 1)``, zero where
    ``x <= th`` (``loudness.py:108-129``)."""

    half = F["loudness_half"]
    loud = (F["loudness_threshold_scale"] * threshs) ** exp * (
        (half + half * pow_dens / threshs) ** exp - F["loudness_one"]
    )
    loud = torch.where(pow_dens <= threshs, torch.full_like(loud, F["loudness_below_threshold"]), loud)
    return loud * sl


def disturbance(deg_loud, ref_loud):
    """``sign(u) max(|u| - 0.25 min(L_deg, L_ref), 0)`` with ``u = L_deg - L_ref``
    (``loss.py:234-237``)."""

    deadzone = F["deadzone"] * torch.min(deg_loud, ref_loud)
    dist = deg_loud - ref_loud
    return dist.sign() * (dist.abs() - deadzone).clamp(min=0)


def weighted_norm(tensor, width_bark, total_width, p):
    """``W ||w x / W^(1/p)||_p`` over bands ``1..`` (``bark.py:176-195``)."""

    scaled = width_bark * tensor / total_width ** (1 / p)
    return total_width * scaled[:, :, F["norm_first_band"]:].norm(p, dim=2)


def asymmetry_factor(equ_deg, equ_ref):
    """``((equ_deg + 50) / (equ_ref + 50))^1.2``, zero below 3, at most 12
    (``loss.py:243-246``)."""

    off = F["asymm_offset"]
    asc = ((equ_deg + off) / (equ_ref + off)) ** F["asymm_exponent"]
    asc = torch.where(asc < F["asymm_cut"], torch.full_like(asc, F["asymm_cut_value"]), asc)
    return asc.clamp(max=F["asymm_cap"])


def frame_weight(taer):
    """``h = ((taer + 1e5) / 1e7)^0.04`` (``loss.py:251-252``)."""

    return ((taer + F["h_offset"]) / F["h_scale"]) ** F["h_exponent"]


def frame_distances(ref: torch.Tensor, deg: torch.Tensor, c=None):
    """Per frame clamped disturbances ``(symm, asymm)`` of ``loss.py:204-253``
    (``reference.py:196-248``)."""

    c = constants() if c is None else c
    th, ex, wb, tw = c["threshs"], c["exp"], c["width_bark"], c["total_width"]

    silent = silent_frames(ref, th)
    ratio = band_ratio(band_means(ref, th, silent), band_means(deg, th, silent))
    equ_ref = ratio.unsqueeze(1) * ref

    taer = total_audible(equ_ref, th, F["total_threshold_factor"])
    tad = total_audible(deg, th, F["total_threshold_factor"])
    equ_deg = frame_ratio(taer, tad).unsqueeze(2) * deg

    dist = disturbance(loudness(equ_deg, th, ex, SL), loudness(equ_ref, th, ex, SL))

    floor, cap = F["distance_floor"], F["distance_cap"]
    symm = weighted_norm(dist, wb, tw, F["symm_norm_p"]).clamp(min=floor)
    asc = asymmetry_factor(equ_deg, equ_ref)
    asymm = weighted_norm(dist * asc, wb, tw, F["asymm_norm_p"]).clamp(min=floor)

    h = frame_weight(taer)
    return (symm / h).clamp(max=cap), (asymm / h).clamp(max=cap)


def overlapping_sums(frames: torch.Tensor) -> torch.Tensor:
    """6th power means over windows of 20 frames at stride 10, then the RMS
    over the windows (``loss.py:255-266``)."""

    power = F["psqm_power"]
    windows = frames.unfold(1, WINDOW, STRIDE)
    psqm = (windows**power).mean(dim=2) ** (1.0 / power)
    return psqm.square().mean(dim=1).sqrt()


def chain(ref: torch.Tensor, deg: torch.Tensor, c=None):
    """Distances ``(d_symm, d_asymm)`` of two Bark spectrograms (``reference.py:159-260``)."""

    symm, asymm = frame_distances(ref.double(), deg.double(), c)
    return overlapping_sums(symm), overlapping_sums(asymm)


def epilogue(d_symm: torch.Tensor, d_asymm: torch.Tensor, factor: float):
    """MOS curve and loss (``loss.py:292-295,322``)."""

    ws, wa = F["pesq_symm_weight"], F["pesq_asymm_weight"]
    inner = F["pesq_offset"] - ws * d_symm - wa * d_asymm
    mos = F["mos_floor"] + F["mos_span"] / (1 + torch.exp(-F["mos_slope"] * inner + F["mos_shift"]))
    return mos, factor * (ws * d_symm + wa * d_asymm)


def pipeline(ref: torch.Tensor, deg: torch.Tensor, sample_rate: int = 16000, c=None):
    """``PesqLoss.raw`` in float64: returns ``(d_symm, d_asymm)``.

    Inputs may require grad; gradients flow through every stage (the peak
    included, whose contribution is analytically zero by scale invariance).
    """

    c = constants() if c is None else c
    ref, deg = torch.atleast_2d(ref).double(), torch.atleast_2d(deg).double()
    ref, deg, _ = peak_normalize(ref, deg)

    if sample_rate != 16000:
        ref, deg = resample(ref, sample_rate), resample(deg, sample_rate)

    ref, deg = align_level(ref, c), align_level(deg, c)
    ref, deg = preemphasize(ref, c), preemphasize(deg, c)

    return chain(stft_bark(ref, c), stft_bark(deg, c), c)
