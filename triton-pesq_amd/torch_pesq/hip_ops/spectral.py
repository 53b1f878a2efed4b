"""HIP STFT + Bark operator (``TritonStftBark``, ``torch_pesq/triton_ops/spectral.py:584-774``).

Forward: per frame a 512 point real FFT (wavefront-per-frame radix-4 Stockham
FFT256 in LDS, float64 arithmetic), |X|^2 with the DC bin dropped, Bark band
sums times the power density correction.  Backward: spectra recomputed, the
adjoint through an inverse FFT of ``gP X``, overlap-add gather (no atomics).
Only the PESQ geometry (``n_fft = 512``, ``hop_length = 256``, 49 bands of a
binary, contiguous filterbank) is supported.
"""

import numpy as np
import torch

from .. import _lib
from ._common import check_input
from .pipeline import pack_model_table

__all__ = ["HipStftBark", "bark_segments"]


def bark_segments(fbank: torch.Tensor):
    """Start / end bin of every band of a binary, contiguous, sorted filterbank.

    Raises ``ValueError`` otherwise (``spectral.py:138-202``).
    """

    mat = fbank.detach().cpu().numpy()
    if mat.ndim != 2:
        raise ValueError(f"The filterbank has to be 2d, got {mat.ndim} dimensions.")
    if not np.all((mat == 0.0) | (mat == 1.0)):
        raise ValueError("The HIP spectral op needs a binary filterbank.")
    nbarks, nfreqs = mat.shape
    starts, ends = np.zeros(nbarks, dtype=np.int64), np.zeros(nbarks, dtype=np.int64)
    prev = 0
    for band in range(nbarks):
        nz = np.flatnonzero(mat[band])
        if nz.size == 0:
            starts[band] = ends[band] = prev
            continue
        start, end = int(nz[0]), int(nz[-1]) + 1
        if end - start != nz.size:
            raise ValueError(f"Band {band} of the filterbank is not contiguous.")
        if start < prev:
            raise ValueError(f"Band {band} starts at bin {start} but the previous band ends at {prev}.")
        starts[band], ends[band] = start, end
        prev = end
    return starts, ends


class _StftBarkFunction(torch.autograd.Function):
    @staticmethod
    def forward(ctx, signal, module, n_padded):
        rows, length = signal.shape
        frames = 1 + (n_padded - module.n_fft) // module.hop_length
        out = torch.empty((rows, frames, module.nbarks), device=signal.device)
        lib = _lib.library()
        with torch.cuda.device(signal.device):
            _lib.check(
                lib.pesq_stft_bark_forward(_lib.ptr(signal), rows, length, n_padded,
                                           _lib.ptr(module.table), _lib.ptr(out),
                                           _lib.stream_handle(signal.device)),
                "pesq_stft_bark_forward",
            )
        ctx.save_for_backward(signal)
        ctx.module, ctx.n_padded = module, n_padded
        return out

    @staticmethod
    @torch.autograd.function.once_differentiable
    def backward(ctx, grad):
        (signal,) = ctx.saved_tensors
        if not ctx.needs_input_grad[0]:
            return None, None, None
        grad = grad.contiguous().float()
        rows, length = signal.shape
        g_x = torch.empty_like(signal)
        lib = _lib.library()
        with torch.cuda.device(signal.device):
            _lib.check(
                lib.pesq_stft_bark_backward(_lib.ptr(grad), _lib.ptr(signal), rows, length,
                                            ctx.n_padded, _lib.ptr(ctx.module.table), _lib.ptr(g_x),
                                            _lib.stream_handle(signal.device)),
                "pesq_stft_bark_backward",
            )
        return g_x, None, None


class HipStftBark(torch.nn.Module):
    """Fused STFT, power spectrum and Bark band aggregation.

    Numerically ``torch.stft(center=False)``, ``|X|**2``, DC bin dropped, a
    contraction with the binary Bark filterbank over bins ``0 .. n_fft/2 - 1``
    and the power density correction (``reference.py:79-127``), evaluated
    with a float64 FFT and returned in float32.
    """

    def __init__(self, window, fbank, pow_dens_correction, n_fft: int = 512, hop_length: int = 256):
        super().__init__()
        if n_fft != 512 or hop_length != 256:
            raise ValueError(
                f"The HIP spectral op supports n_fft=512 and hop_length=256, got {n_fft} and {hop_length}."
            )
        if window.ndim != 1 or window.shape[0] > n_fft:
            raise ValueError(f"The window has to be 1d with at most {n_fft} taps, got {tuple(window.shape)}.")
        if fbank.shape[1] != n_fft // 2:
            raise ValueError(f"The filterbank needs {n_fft // 2} bins, got {fbank.shape[1]}.")
        if pow_dens_correction.shape[0] != fbank.shape[0]:
            raise ValueError("The power density correction needs one entry per band.")
        if fbank.shape[0] != _lib.NBARKS:
            raise ValueError(f"The HIP spectral op needs {_lib.NBARKS} bands, got {fbank.shape[0]}.")
        self.starts, self.ends = bark_segments(fbank)
        self.n_fft, self.hop_length, self.nbarks = n_fft, hop_length, fbank.shape[0]
        full = torch.zeros(n_fft)
        left = (n_fft - window.shape[0]) // 2
        full[left : left + window.shape[0]] = window.detach().cpu().float()
        ones = torch.ones(_lib.NBARKS, dtype=torch.float64)
        table = pack_model_table(None, None, None, None, full, fbank, pow_dens_correction,
                                 ones, ones, ones, 1.0, 0.0)
        self.register_buffer("window", full)
        self.register_buffer("table", table, persistent=False)

    def forward(self, signal: torch.Tensor, n_padded: int = None) -> torch.Tensor:
        """Bark scaled power spectrogram ``[batch, frame, bark]`` of ``[batch, sample]``."""

        signal = check_input(signal, "signal")
        if signal.ndim != 2:
            raise ValueError(f"`signal` has to be 2d, got {signal.ndim} dimensions instead.")
        n_padded = signal.shape[1] if n_padded is None else int(n_padded)
        if n_padded < signal.shape[1]:
            raise ValueError(f"`n_padded` ({n_padded}) is smaller than the signal length ({signal.shape[1]}).")
        if n_padded < self.n_fft:
            raise ValueError(f"`n_padded` ({n_padded}) is shorter than one frame ({self.n_fft}).")
        if self.table.device != signal.device:
            raise RuntimeError(f"The module lives on {self.table.device} but the signal on {signal.device}.")
        return _StftBarkFunction.apply(signal, self, n_padded)
