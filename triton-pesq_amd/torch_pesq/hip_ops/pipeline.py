"""Host calls of the fused PESQ pipeline.

Forward: ``pesq_pipeline_forward`` (five kernels) evaluates, for 16 kHz rows,
everything ``PesqLossTriton.raw`` + ``mos`` + ``forward`` compute in the
reference (``torch_pesq/triton_ops/loss.py:104-147,203-215``): peak
normalisation, level alignment, pre-emphasis, STFT, Bark, the perceptual chain
and the MOS epilogue.  Backward: ``pesq_pipeline_backward`` (four kernels).

The forward workspace carries the state the backward reads (the filtered and
pre-emphasised signals, Bark spectra, chain intermediates).  The autograd node
that saves it between the two calls is C++ (``csrc/torch_autograd.cpp``,
reached through ``_lib.torch_ext().pipeline``), so that the backward runs no
Python on autograd's worker thread; the functions here make the same two calls
from Python for measurement and the stage tests.
"""

import ctypes

import numpy as np
import torch

from .. import _lib
from .iir import parallel_sections, sections_struct

__all__ = [
    "pack_model_table",
    "pipeline_forward",
    "pipeline_backward",
    "pipeline_region",
]


def pack_model_table(
    power_b, power_a, pre_b, pre_a, window, fbank, corr, threshs, exps, width, total_width, sl
) -> torch.Tensor:
    """Pack the model constants into the library's device table (host bytes).

    ``power_b`` / ``pre_b`` may be ``None`` (both), giving a table for the
    stand-alone STFT and chain operators only.
    """

    constants = _lib.ModelConstants()
    if power_b is not None:
        c0, secs = parallel_sections(power_b, power_a)
        constants.power_filter = sections_struct(c0, secs)
        c0, secs = parallel_sections(pre_b, pre_a)
        constants.pre_filter = sections_struct(c0, secs)

    window = torch.as_tensor(window).detach().cpu().float().numpy()
    if window.shape != (_lib.NFFT,):
        raise ValueError(f"The HIP pipeline needs a {_lib.NFFT} tap window, got {window.shape}.")
    constants.window[:] = window.tolist()

    mat = torch.as_tensor(fbank).detach().cpu().double().numpy()
    if mat.shape != (_lib.NBARKS, _lib.NFFT // 2):
        raise ValueError(f"The HIP pipeline needs a [49, 256] filterbank, got {mat.shape}.")
    if not np.all((mat == 0.0) | (mat == 1.0)):
        raise ValueError("The HIP pipeline needs a binary filterbank.")
    prev = 0
    for band in range(mat.shape[0]):
        nz = np.flatnonzero(mat[band])
        start, end = (prev, prev) if nz.size == 0 else (int(nz[0]), int(nz[-1]) + 1)
        if nz.size and (end - start != nz.size or start < prev):
            raise ValueError(f"Band {band} of the filterbank is not contiguous and sorted.")
        constants.band_start[band], constants.band_end[band] = start, end
        prev = end

    def fill(dst, values):
        values = torch.as_tensor(values).detach().cpu().double().reshape(-1).numpy()
        if values.shape != (_lib.NBARKS,):
            raise ValueError(f"Expected {_lib.NBARKS} band values, got {values.shape}.")
        dst[:] = values.tolist()

    fill(constants.corr, corr)
    fill(constants.threshs, threshs)
    fill(constants.exps, exps)
    fill(constants.width, width)
    constants.total_width = float(total_width)
    constants.sl = float(sl)
    constants.nbarks, constants.n_fft, constants.hop = _lib.NBARKS, _lib.NFFT, 256

    lib = _lib.library()
    buf = (ctypes.c_ubyte * lib.pesq_model_table_bytes())()
    _lib.check(lib.pesq_model_table_pack(ctypes.byref(constants), buf), "pesq_model_table_pack")
    return torch.frombuffer(bytearray(buf), dtype=torch.uint8).clone()


def pipeline_region(batch: int, length: int, grad_mask: int, name: str):
    """``(offset, bytes)`` of a named region of the forward workspace."""

    lib = _lib.library()
    off, size = ctypes.c_size_t(0), ctypes.c_size_t(0)
    _lib.check(
        lib.pesq_pipeline_region(
            batch, length, grad_mask, name.encode(), ctypes.byref(off), ctypes.byref(size)
        ),
        "pesq_pipeline_region",
    )
    return int(off.value), int(size.value)


def pipeline_forward(ref, deg, table, factor, grad_mask):
    """Run the forward kernels; returns ``([d_symm, d_asymm, mos, loss], workspace)``.

    The workspace holds the state :func:`pipeline_backward` needs (regions:
    :func:`pipeline_region`).
    """

    lib = _lib.library()
    batch, length = ref.shape
    ws_bytes = _lib.size_query(lib.pesq_pipeline_forward_workspace, batch, length, grad_mask)
    workspace = torch.empty(ws_bytes, dtype=torch.uint8, device=ref.device)
    out = [torch.empty(batch, dtype=torch.float32, device=ref.device) for _ in range(4)]
    with torch.cuda.device(ref.device):
        _lib.check(
            lib.pesq_pipeline_forward(
                _lib.ptr(ref),
                _lib.ptr(deg),
                batch,
                length,
                _lib.ptr(table),
                float(factor),
                grad_mask,
                _lib.ptr(out[0]),
                _lib.ptr(out[1]),
                _lib.ptr(out[2]),
                _lib.ptr(out[3]),
                _lib.ptr(workspace),
                _lib.stream_handle(ref.device),
            ),
            "pesq_pipeline_forward",
        )
    return out, workspace


def pipeline_backward(grads, workspace, table, batch, length, factor, grad_mask):
    """Run the backward kernels; returns ``(g_ref, g_deg)`` (``None`` if not requested)."""

    lib = _lib.library()
    device = workspace.device
    grads = [None if g is None else g.contiguous().float() for g in grads]
    bw_bytes = _lib.size_query(lib.pesq_pipeline_backward_workspace, batch, length, grad_mask)
    scratch = torch.empty(bw_bytes, dtype=torch.uint8, device=device)
    g_ref = g_deg = None
    if grad_mask & _lib.GRAD_REF:
        g_ref = torch.empty((batch, length), dtype=torch.float32, device=device)
    if grad_mask & _lib.GRAD_DEG:
        g_deg = torch.empty((batch, length), dtype=torch.float32, device=device)
    with torch.cuda.device(device):
        _lib.check(
            lib.pesq_pipeline_backward(
                *[_lib.ptr(g) for g in grads],
                batch,
                length,
                _lib.ptr(table),
                float(factor),
                grad_mask,
                _lib.ptr(g_ref),
                _lib.ptr(g_deg),
                _lib.ptr(workspace),
                _lib.ptr(scratch),
                _lib.stream_handle(device),
            ),
            "pesq_pipeline_backward",
        )
    return g_ref, g_deg
