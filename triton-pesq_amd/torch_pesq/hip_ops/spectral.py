"""HIP STFT + Bark operator (``TritonStftBark``, ``torch_pesq/triton_ops/spectral.py:584-774``).

Forward: per frame a real FFT of the windowed frame in float64, |X|^2 with
the DC bin dropped, Bark band sums times the power density correction.
Backward: spectra recomputed, the adjoint through an inverse FFT of
``gP X``, overlap-add gather (no atomics).

Two kernel families serve it: the PESQ geometry (``n_fft = 512``,
``hop_length = 256``, 49 bands of at most 25 bins) runs the specialised
radix-4 kernels of ``csrc/pipeline.hip``; every other geometry, i.e.
``n_fft`` a power of two in [32, 1024], any ``hop_length`` (also longer than
``n_fft``, where uncovered samples get a zero gradient), windows shorter than
``n_fft`` (centred like ``torch.stft``) and up to 128 bands, runs the general
radix-2 kernels of ``csrc/stft_generic.hip``.
"""

import ctypes

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
            raise ValueError(
                f"Band {band} starts at bin {start} but the previous band ends at {prev}; "
                "the bands have to be disjoint and sorted."
            )
        starts[band], ends[band] = start, end
        prev = end
    return starts, ends


def _general_table(window, starts, ends, corr, n_fft, hop) -> torch.Tensor:
    lib = _lib.library()
    win = np.ascontiguousarray(window.detach().cpu().numpy(), dtype=np.float32)
    lo = np.ascontiguousarray(starts, dtype=np.int32)
    hi = np.ascontiguousarray(ends, dtype=np.int32)
    cor = np.ascontiguousarray(corr.detach().cpu().double().numpy(), dtype=np.float64)
    buf = (ctypes.c_ubyte * lib.pesq_stft_table_bytes())()
    _lib.check(
        lib.pesq_stft_table_pack(
            n_fft, hop, win.ctypes.data_as(ctypes.c_void_p), lo.shape[0],
            lo.ctypes.data_as(ctypes.c_void_p), hi.ctypes.data_as(ctypes.c_void_p),
            cor.ctypes.data_as(ctypes.c_void_p), buf,
        ),
        "pesq_stft_table_pack",
    )
    return torch.frombuffer(bytearray(buf), dtype=torch.uint8).clone()


class _StftBarkFunction(torch.autograd.Function):
    @staticmethod
    def forward(ctx, signal, module, n_padded):
        rows, length = signal.shape
        frames = 1 + (n_padded - module.n_fft) // module.hop_length
        out = torch.empty((rows, frames, module.nbarks), device=signal.device)
        lib = _lib.library()
        stream = _lib.stream_handle(signal.device)
        with torch.cuda.device(signal.device):
            if module.general:
                status = lib.pesq_stft_forward(
                    _lib.ptr(signal), rows, length, n_padded, _lib.ptr(module.table),
                    module.n_fft, module.hop_length, module.nbarks, _lib.ptr(out), stream)
                _lib.check(status, "pesq_stft_forward")
            else:
                status = lib.pesq_stft_bark_forward(
                    _lib.ptr(signal), rows, length, n_padded, _lib.ptr(module.table),
                    _lib.ptr(out), stream)
                _lib.check(status, "pesq_stft_bark_forward")
        ctx.save_for_backward(signal)
        ctx.module, ctx.n_padded = module, n_padded
        return out

    @staticmethod
    @torch.autograd.function.once_differentiable
    def backward(ctx, grad):
        (signal,) = ctx.saved_tensors
        if not ctx.needs_input_grad[0]:
            return None, None, None
        module = ctx.module
        grad = grad.contiguous().float()
        rows, length = signal.shape
        g_x = torch.empty_like(signal)
        lib = _lib.library()
        stream = _lib.stream_handle(signal.device)
        with torch.cuda.device(signal.device):
            if module.general:
                size = _lib.size_query(lib.pesq_stft_workspace, rows, length, ctx.n_padded,
                                       module.n_fft, module.hop_length)
                scratch = torch.empty(max(size, 4), dtype=torch.uint8, device=signal.device)
                status = lib.pesq_stft_backward(
                    _lib.ptr(grad), _lib.ptr(signal), rows, length, ctx.n_padded,
                    _lib.ptr(module.table), module.n_fft, module.hop_length, module.nbarks,
                    _lib.ptr(g_x), _lib.ptr(scratch), stream)
                _lib.check(status, "pesq_stft_backward")
            else:
                status = lib.pesq_stft_bark_backward(
                    _lib.ptr(grad), _lib.ptr(signal), rows, length, ctx.n_padded,
                    _lib.ptr(module.table), _lib.ptr(g_x), stream)
                _lib.check(status, "pesq_stft_bark_backward")
        return g_x, None, None


#: geometry of the specialised kernels
_PESQ_GEOMETRY = (512, 256, _lib.NBARKS)
_MAX_BAND_BINS = 25
_MAX_BANDS = 128


class HipStftBark(torch.nn.Module):
    """Fused STFT, power spectrum and Bark band aggregation.

    Numerically ``torch.stft(center=False)``, ``|X|**2``, DC bin dropped, a
    contraction with the binary Bark filterbank over bins ``0 .. n_fft/2 - 1``
    and the power density correction (``reference.py:79-127``), evaluated
    with a float64 FFT and returned in float32.  Same constructor and
    validation as ``TritonStftBark`` (``spectral.py:584-700``).

    Attributes
    ----------
    general : bool
        The configuration runs the general kernels (anything but the PESQ
        geometry)
    novertaps : int
        Frames a sample belongs to at most, ``ceil(n_fft / hop_length)``
    """

    def __init__(self, window, fbank, pow_dens_correction, n_fft: int = 512, hop_length: int = 256):
        super().__init__()
        n_fft, hop_length = int(n_fft), int(hop_length)
        if n_fft < 32:
            raise ValueError(f"`n_fft` has to be at least 32, got {n_fft}.")
        half = n_fft // 2
        if n_fft % 2 or half & (half - 1):
            raise ValueError(f"`n_fft // 2` has to be a power of two, got n_fft = {n_fft}.")
        if n_fft > 1024:
            raise ValueError(f"`n_fft` can be at most 1024 (512 bins), got {n_fft}.")
        if hop_length < 1:
            raise ValueError(f"`hop_length` has to be positive, got {hop_length}.")
        if window.ndim != 1 or window.shape[0] > n_fft:
            raise ValueError(
                f"The window has to be 1d with at most {n_fft} taps, got {tuple(window.shape)}."
            )
        if fbank.ndim != 2 or fbank.shape[1] != half:
            raise ValueError(
                f"The filterbank needs n_fft // 2 = {half} bins, got {tuple(fbank.shape)}."
            )
        if pow_dens_correction.reshape(-1).shape[0] != fbank.shape[0]:
            raise ValueError("The power density correction needs one entry per band.")
        if fbank.shape[0] > _MAX_BANDS:
            raise ValueError(f"At most {_MAX_BANDS} bands are supported, got {fbank.shape[0]}.")
        self.starts, self.ends = bark_segments(fbank)
        self.n_fft, self.hop_length, self.nbarks = n_fft, hop_length, fbank.shape[0]
        self.novertaps = -(-n_fft // hop_length)
        full = torch.zeros(n_fft)
        left = (n_fft - window.shape[0]) // 2
        full[left : left + window.shape[0]] = window.detach().cpu().float()
        corr = pow_dens_correction.reshape(-1)
        self.general = (n_fft, hop_length, self.nbarks) != _PESQ_GEOMETRY or bool(
            np.any(self.ends - self.starts > _MAX_BAND_BINS)
        )
        if self.general:
            table = _general_table(full, self.starts, self.ends, corr, n_fft, hop_length)
        else:
            ones = torch.ones(_lib.NBARKS, dtype=torch.float64)
            table = pack_model_table(None, None, None, None, full, fbank, corr,
                                     ones, ones, ones, 1.0, 0.0)
        self.register_buffer("window", full)
        self.register_buffer("correction", corr.detach().clone().float())
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
