"""Windowed sinc resampling bank, torchaudio's published design restated.

The reference takes its resampling kernel from torchaudio
(``_get_sinc_resample_kernel``, called at ``triton_ops/resample.py:512-521``
and through ``torchaudio.transforms.Resample`` at ``loss.py:76``).  torchaudio
is a third party dependency that is not installed here, so the design is
restated from its published algorithm; it has to produce the same taps, which
is why the steps below follow it one for one.
"""

import math

import torch

__all__ = ["sinc_resample_kernel", "resample_length"]


def sinc_resample_kernel(
    orig_freq: int,
    new_freq: int,
    lowpass_filter_width: int = 6,
    rolloff: float = 0.99,
    resampling_method: str = "sinc_interp_hann",
    beta=None,
):
    """Filter bank ``[new_step, width_total]`` (float32) and the pad ``width``.

    With both rates divided by their gcd, ``base = min(orig, new) * rolloff``,
    ``width = ceil(lpw * orig / base)``; for phase ``j`` and tap ``k``
    ``t = (-j / new + (k - width) / orig) * base`` clamped to ``[-lpw, lpw]``
    and the tap is ``sinc(pi t) * window(t) * base / orig``, the window being
    ``cos(pi t / (2 lpw)) ** 2`` (Hann) or a Kaiser window.  The phase term is
    a float32 division (an integer ``arange`` divided by ``new``), the rest is
    float64, and the bank is rounded to float32.
    """

    if int(orig_freq) != orig_freq or int(new_freq) != new_freq:
        raise ValueError("Frequencies must be integers.")
    if resampling_method in ("sinc_interpolation", "kaiser_window"):
        resampling_method = {
            "sinc_interpolation": "sinc_interp_hann",
            "kaiser_window": "sinc_interp_kaiser",
        }[resampling_method]
    if resampling_method not in ("sinc_interp_hann", "sinc_interp_kaiser"):
        raise ValueError(f"Invalid resampling method: {resampling_method}")
    if lowpass_filter_width <= 0:
        raise ValueError("Low pass filter width should be positive.")

    gcd = math.gcd(int(orig_freq), int(new_freq))
    orig, new = int(orig_freq) // gcd, int(new_freq) // gcd
    base = min(orig, new) * rolloff
    width = math.ceil(lowpass_filter_width * orig / base)

    idx = torch.arange(-width, width + orig, dtype=torch.float64)[None, None] / orig
    t = torch.arange(0, -new, -1)[:, None, None] / new + idx
    t = (t * base).clamp(-lowpass_filter_width, lowpass_filter_width)

    if resampling_method == "sinc_interp_hann":
        window = torch.cos(t * math.pi / lowpass_filter_width / 2) ** 2
    else:
        beta = 14.769656459379492 if beta is None else beta
        beta_t = torch.tensor(float(beta))
        window = torch.i0(beta_t * torch.sqrt(1 - (t / lowpass_filter_width) ** 2)) / torch.i0(beta_t)

    t = t * math.pi
    taps = torch.where(t == 0, torch.tensor(1.0, dtype=t.dtype), t.sin() / t)
    taps = taps * window * (base / orig)
    return taps.to(torch.float32).reshape(new, -1), width


def resample_length(n_samples: int, orig_step: int, new_step: int) -> int:
    """Output length: ``ceil(new * n / orig)`` evaluated in float32 (``resample.py:269-277``)."""

    return int(torch.ceil(torch.as_tensor(new_step * n_samples / orig_step, dtype=torch.float32)).long())
