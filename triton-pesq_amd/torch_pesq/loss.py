"""PESQ loss evaluated by HIP kernels on an AMD Instinct GPU.

:class:`PesqLoss` keeps the constructor, attributes and methods of the
reference ``torch_pesq/loss.py:20-322`` (``raw``, ``mos``, ``forward``,
``align_level``, ``preemphasize``; ``resampler``, ``to_spec``, ``fbank``,
``loudness``, ``power_filter``, ``pre_filter``).  Every computation runs on
the GPU through ``libpesq_hip.so``; CPU tensors are rejected with a
``RuntimeError``.

``raw``/``mos``/``forward`` go through the fused pipeline (``csrc/pipeline.hip``)
at the PESQ geometry (49 bands, ``n_fft = win_length = 512``,
``hop_length = 256``).  Other STFT geometries (``n_fft``, ``win_length``,
``hop_length``) run the reference's stage sequence (``triton_ops/loss.py:104-147``)
on the stand-alone operators, with the general STFT kernels.  ``align_level``
and ``preemphasize`` are the stand-alone per stage operators.
"""

import numpy as np
import torch
from scipy.signal import butter
from torch.nn import Parameter

from .bark import BarkScale
from .loudness import Loudness, Sl_16k

__all__ = ["PesqLoss", "SpectrogramSpec"]

#: loudness calibration constant used by the perceptual chain
#: (``torch_pesq/triton_ops/reference.py:322``; ``loudness.py:Sl_16k``)
SL = 0.1866055


class SpectrogramSpec(torch.nn.Module):
    """Parameters of the framed power spectrogram (``loss.py:79-87``).

    ``torch.hann_window(win_length)`` (periodic, float32), centred into
    ``n_fft`` taps, power 2, no centring of the frames, no normalisation.
    """

    def __init__(self, win_length: int = 512, n_fft: int = 512, hop_length: int = 256):
        super().__init__()
        self.n_fft = int(n_fft)
        self.win_length = int(win_length)
        self.hop_length = int(hop_length)
        if self.win_length > self.n_fft:
            raise ValueError(f"win_length {win_length} exceeds n_fft {n_fft}.")
        window = torch.zeros(self.n_fft, dtype=torch.float32)
        left = (self.n_fft - self.win_length) // 2
        window[left : left + self.win_length] = torch.hann_window(self.win_length)
        self.register_buffer("window", window)


class PesqLoss(torch.nn.Module):
    """Perceptual Evaluation of Speech Quality as a differentiable loss.

    Parameters
    ----------
    factor : float
        Scaling of the loss function
    sample_rate : int
        Sampling rate of the inputs; other rates than 16 kHz are resampled
    nbarks, win_length, n_fft, hop_length : int
        Bark bands and STFT geometry.  The loudness exponents are the
        standard's 49 values (``loudness.py:44-55`` does not interpolate them),
        so ``nbarks != 49`` raises ``ValueError`` like the reference's chain
        does; ``n_fft`` (a power of two in [32, 1024]), ``win_length <=
        n_fft`` and ``hop_length`` are free.
    """

    factor: float

    def __init__(
        self,
        factor: float,
        sample_rate: int = 48000,
        nbarks: int = 49,
        win_length: int = 512,
        n_fft: int = 512,
        hop_length: int = 256,
    ):
        super().__init__()

        from .hip_ops.chain import HipPesqChain
        from .hip_ops.iir import HipIIR
        from .hip_ops.pipeline import pack_model_table
        from .hip_ops.resample import HipResample
        from .hip_ops.spectral import HipStftBark

        self.factor = factor
        self.source_sample_rate = int(sample_rate)

        self.resampler = HipResample(self.source_sample_rate, 16000)
        self.to_spec = SpectrogramSpec(win_length, n_fft, hop_length)
        self.fbank = BarkScale(n_fft // 2, nbarks)
        self.loudness = Loudness(nbarks)

        coeffs = np.asarray(butter(5, [325, 3250], fs=16000, btype="band"))
        self.power_filter = Parameter(torch.as_tensor(coeffs, dtype=torch.float32), requires_grad=False)
        self.pre_filter = Parameter(
            torch.tensor(
                [[2.740826, -5.4816519, 2.740826], [1.0, -1.9444777, 0.94597794]],
                dtype=torch.float32,
            ),
            requires_grad=False,
        )

        # stand-alone per stage operators (align_level / preemphasize)
        self.power_iir = HipIIR(self.power_filter[0], self.power_filter[1])
        self.pre_iir = HipIIR(self.pre_filter[0], self.pre_filter[1])

        # the per stage operators of the general geometry (triton_ops/loss.py:75-92)
        self.general = (nbarks, win_length, n_fft, hop_length) != (49, 512, 512, 256)
        self.spectral = HipStftBark(
            self.to_spec.window,
            self.fbank.fbank,
            self.fbank.pow_dens_correction,
            n_fft,
            hop_length,
        )
        self.chain = HipPesqChain(
            self.loudness.threshs.flatten(),
            self.loudness.exp.flatten(),
            self.fbank.width_bark,
            float(self.fbank.total_width),
            SL,
        )
        if self.general:
            self.register_buffer("model_table", self.spectral.table, persistent=False)
            return

        table = pack_model_table(
            self.power_filter[0],
            self.power_filter[1],
            self.pre_filter[0],
            self.pre_filter[1],
            self.to_spec.window,
            self.fbank.fbank,
            self.fbank.pow_dens_correction,
            self.loudness.threshs,
            self.loudness.exp,
            self.fbank.width_bark,
            self.fbank.total_width,
            SL,
        )
        self.register_buffer("model_table", table, persistent=False)

    # -- stages -------------------------------------------------------------

    def align_level(self, signal: torch.Tensor) -> torch.Tensor:
        """Align the 325 Hz - 3.25 kHz band power of ``signal`` to 1e7 (``loss.py:111-141``)."""

        from .hip_ops.elementwise import align_scale

        return align_scale(signal, self.power_iir(signal))

    def preemphasize(self, signal: torch.Tensor) -> torch.Tensor:
        """Edge ramp and pre-emphasis filter (``loss.py:144-169``)."""

        from .hip_ops.elementwise import edge_ramp

        return self.pre_iir(edge_ramp(signal))

    # -- pipeline -----------------------------------------------------------

    def _run(self, ref: torch.Tensor, deg: torch.Tensor):
        from . import _lib
        from .hip_ops._common import check_input

        deg, ref = torch.atleast_2d(deg), torch.atleast_2d(ref)
        if ref.shape != deg.shape:
            raise ValueError(
                "Reference and degraded signal must have the same shape, "
                f"got {tuple(ref.shape)} and {tuple(deg.shape)}."
            )
        if ref.dim() != 2:
            raise ValueError(f"Expected [batch, sample] signals, got {tuple(ref.shape)}.")
        ref = check_input(ref, "ref")
        deg = check_input(deg, "deg")
        if self.model_table.device != ref.device:
            raise RuntimeError(
                f"The module lives on {self.model_table.device} but the signals on "
                f"{ref.device}; move it with `.to(...)` first."
            )

        if self.general:
            return self._run_stages(ref, deg)

        resampled = self.source_sample_rate != 16000
        if resampled:
            if self.resampler.kernel.device != ref.device:
                raise RuntimeError(
                    f"The resampling kernel lives on {self.resampler.kernel.device} but the "
                    f"signals on {ref.device}, move the module with `.to(...)`."
                )
            length = self.resampler.output_length(ref.shape[1])
            self.resampler.check_length(ref.shape[1], length)
        else:
            length = ref.shape[1]
        padded = length + length % 256
        frames = 1 + (padded - 512) // 256 if padded >= 512 else 0
        if length < 15:
            raise RuntimeError(
                f"The edge ramp needs at least 15 samples at 16 kHz, got {length}."
            )
        if frames < 20:
            raise ValueError(
                "The PESQ chain needs at least 20 frames for the overlapping sums, "
                f"got {frames}."
            )
        if isinstance(self.factor, torch.Tensor) and self.factor.requires_grad:
            raise RuntimeError(
                "The loss treats `factor` as a constant, pass a Python float. A tensor "
                "that requires a gradient would receive none."
            )
        if resampled:
            bank, steps = self.resampler.bank()
            return tuple(
                _lib.torch_ext().pipeline_resampled(
                    ref, deg, self.model_table, float(self.factor), bank, steps, length
                )
            )
        return tuple(_lib.torch_ext().pipeline(ref, deg, self.model_table, float(self.factor)))

    def _run_stages(self, ref: torch.Tensor, deg: torch.Tensor):
        """The stage sequence of ``PesqLossTriton.raw`` (``triton_ops/loss.py:104-147``).

        Both signals share one peak and are stacked into one batch of twice
        the size; resampling, level alignment, pre-emphasis, the ``N % 256``
        padding, the STFT / Bark operator, the chain and the epilogue follow.
        """

        from .hip_ops.elementwise import peak_normalize, pesq_epilogue

        if isinstance(self.factor, torch.Tensor) and self.factor.requires_grad:
            raise RuntimeError(
                "The loss treats `factor` as a constant, pass a Python float. A tensor "
                "that requires a gradient would receive none."
            )
        batch = ref.shape[0]
        signal = peak_normalize(ref, deg, stack=True)
        if self.source_sample_rate != 16000:
            signal = self.resampler(signal)
        length = signal.shape[1]
        if length < 15:
            raise RuntimeError(
                f"The edge ramp needs at least 15 samples at 16 kHz, got {length}."
            )
        padded = length + length % 256
        n_fft, hop = self.to_spec.n_fft, self.to_spec.hop_length
        frames = 1 + (padded - n_fft) // hop if padded >= n_fft else 0
        if frames < 20:
            raise ValueError(
                "The PESQ chain needs at least 20 frames for the overlapping sums, "
                f"got {frames}."
            )
        signal = self.align_level(signal)
        signal = self.preemphasize(signal)
        bark = self.spectral(signal, padded)
        d_symm, d_asymm = self.chain(bark[:batch], bark[batch:])
        mos, loss = pesq_epilogue(d_symm, d_asymm, float(self.factor))
        return d_symm, d_asymm, mos, loss

    def raw(self, ref: torch.Tensor, deg: torch.Tensor):
        """Symmetric and asymmetric distances, both ``[batch]``."""

        d_symm, d_asymm, _, _ = self._run(ref, deg)
        return d_symm, d_asymm

    def mos(self, ref: torch.Tensor, deg: torch.Tensor) -> torch.Tensor:
        """Mean opinion score in ``(1.08, 4.999)`` (``loss.py:271-297``)."""

        return self._run(ref, deg)[2]

    def forward(self, ref: torch.Tensor, deg: torch.Tensor) -> torch.Tensor:
        """Loss ``factor * (0.1 d_symm + 0.0309 d_asymm)`` (``loss.py:300-322``)."""

        return self._run(ref, deg)[3]
