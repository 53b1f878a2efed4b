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
* chain: the identical-input known answer (``1e-20 / h`` floor,
  ``test_triton_chain.py:365-383``), a float64 finite difference check of the
  autograd gradient, and a pure-Python loop evaluation on a tiny spectrum;
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

SL = 0.1866055  # torch_pesq/triton_ops/reference.py:322
WINDOW, STRIDE = 20, 10  # torch_pesq/loss.py:291-298


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

    exp32 = 6 / (torch.tensor(TABLES["centre_of_band_bark_16k"], dtype=torch.float32) + 2.0)
    exp32 = exp32.clamp(min=1.0, max=2.0) ** 0.15 * TABLES["zwicker_power"]

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
    power = (filtered**2).sum(dim=1, keepdim=True) / (filtered.shape[1] + 5120) / 1.04684
    return signal * (10**7 / power).sqrt()


def edge_ramp(signal: torch.Tensor) -> torch.Tensor:
    """First and last 15 samples times ``k/16``, applied in that order (``loss.py:163-165``)."""

    emp = torch.linspace(0, 15, 16, dtype=torch.float32)[1:] / 16.0
    emp = emp.to(signal.dtype)
    out = signal.clone()
    out[:, :15] = out[:, :15] * emp
    out[:, -15:] = out[:, -15:] * torch.flip(emp, dims=(0,))
    return out


def preemphasize(signal: torch.Tensor, c=None) -> torch.Tensor:
    """``loss.py:163-167`` / ``reference.py:54-76``."""

    c = constants() if c is None else c
    return lfilter(edge_ramp(signal), c["pre_b"], c["pre_a"])


def n_frames(n_samples: int, n_fft: int = 512, hop: int = 256) -> int:
    """Frames after the reference's ``length % 256`` padding (``loss.py:191-192``)."""

    padded = n_samples + n_samples % 256
    return 1 + (padded - n_fft) // hop


def stft_bark(signal: torch.Tensor, c=None) -> torch.Tensor:
    """Pad by ``N % 256``, float64 STFT, DC dropped, Bark sums (``reference.py:79-127``)."""

    c = constants() if c is None else c
    signal = torch.nn.functional.pad(signal, (0, signal.shape[1] % 256))
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


def _total_audible(tensor, threshs, factor):
    return (tensor * (tensor > threshs * factor)).sum(dim=2)


def _loudness(pow_dens, threshs, exp, sl):
    loud = (2.0 * threshs) ** exp * ((0.5 + 0.5 * pow_dens / threshs) ** exp - 1)
    loud = torch.where(pow_dens <= threshs, torch.zeros_like(loud), loud)
    return loud * sl


def _weighted_norm(tensor, width_bark, total_width, p):
    return total_width * (width_bark * tensor / total_width ** (1 / p))[:, :, 1:].norm(p, dim=2)


def frame_distances(ref: torch.Tensor, deg: torch.Tensor, c=None):
    """Per frame clamped disturbances ``(symm, asymm)`` of ``reference.py:196-248``."""

    c = constants() if c is None else c
    th, ex, wb, tw = c["threshs"], c["exp"], c["width_bark"], c["total_width"]

    silent = _total_audible(ref, th, 1e2) < 1e7
    mask_ref = (ref > th * 100.0) * (~silent.unsqueeze(2))
    mask_deg = (deg > th * 100.0) * (~silent.unsqueeze(2))
    mean_ref = (ref * mask_ref).mean(dim=1)
    mean_deg = (deg * mask_deg).mean(dim=1)

    ratio = ((mean_deg + 1000) / (mean_ref + 1000)).unsqueeze(1).clamp(min=0.01, max=100.0)
    equ_ref = ratio * ref

    taer = _total_audible(equ_ref, th, 1.0)
    fpr = (taer + 5e3) / (_total_audible(deg, th, 1.0) + 5e3)
    fpr = torch.cat([fpr[:, :1], fpr[:, 1:] * 0.8 + fpr[:, :-1] * 0.2], dim=1)
    fpr = fpr.clamp(min=3e-4, max=5.0)
    equ_deg = fpr.unsqueeze(2) * deg

    deg_loud = _loudness(equ_deg, th, ex, SL)
    ref_loud = _loudness(equ_ref, th, ex, SL)

    deadzone = 0.25 * torch.min(deg_loud, ref_loud)
    dist = deg_loud - ref_loud
    dist = dist.sign() * (dist.abs() - deadzone).clamp(min=0)

    symm = _weighted_norm(dist, wb, tw, 2.0).clamp(min=1e-20)

    asc = ((equ_deg + 50.0) / (equ_ref + 50.0)) ** 1.2
    asc = torch.where(asc < 3.0, torch.zeros_like(asc), asc).clamp(max=12.0)
    asymm = _weighted_norm(dist * asc, wb, tw, 1.0).clamp(min=1e-20)

    h = ((taer + 1e5) / 1e7) ** 0.04
    return (symm / h).clamp(max=45.0), (asymm / h).clamp(max=45.0)


def overlapping_sums(frames: torch.Tensor) -> torch.Tensor:
    """6th power means over windows of 20 frames at stride 10, then the RMS."""

    windows = frames.unfold(1, WINDOW, STRIDE)
    psqm = (windows**6).mean(dim=2) ** (1.0 / 6)
    return psqm.square().mean(dim=1).sqrt()


def chain(ref: torch.Tensor, deg: torch.Tensor, c=None):
    """Distances ``(d_symm, d_asymm)`` of two Bark spectrograms (``reference.py:159-260``)."""

    symm, asymm = frame_distances(ref.double(), deg.double(), c)
    return overlapping_sums(symm), overlapping_sums(asymm)


def epilogue(d_symm: torch.Tensor, d_asymm: torch.Tensor, factor: float):
    """MOS curve and loss (``loss.py:292-295,322``)."""

    inner = 4.5 - 0.1 * d_symm - 0.0309 * d_asymm
    mos = 0.999 + 4 / (1 + torch.exp(-1.3669 * inner + 3.8224))
    return mos, factor * (0.1 * d_symm + 0.0309 * d_asymm)


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
