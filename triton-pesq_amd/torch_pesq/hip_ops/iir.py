"""HIP IIR filter, the ``TritonIIR`` operator (``torch_pesq/triton_ops/iir.py:1266-1482``).

Realisation
-----------
The difference equation ``b / a`` is realised in *parallel form*: the partial
fraction expansion (``scipy.signal.residuez``) gives a direct term ``c0`` and
one residue per pole; conjugate pole pairs, and pairs of real poles, are
merged into second order sections

    H(z) = c0 + sum_k (b0_k + b1_k z^-1) / (1 + a1_k z^-1 + a2_k z^-2)

Every section is evaluated as a direct form II transposed biquad with a
float64 state, so the chunk transfer matrices of the scan are 2x2 blocks (see
``csrc/iir.hpp``).  Filters of order <= 2 are used as a single section as
given.  The realisation is checked against the float64 impulse response of the
difference equation; a filter that cannot be realised this way (repeated
poles, more numerator than denominator terms beyond the direct feed through)
raises, mirroring the reference's refusal of filters it cannot represent
(``iir.py:580-597``).

Backward
--------
The filter is a lower triangular Toeplitz operator T, so its adjoint is
J T J (J = time reversal): the same filter run over the reversed signal.  The
kernels do the reversal by index, like the reference (``iir.py:1232-1258``).
"""

import ctypes
import math
import warnings
from typing import Optional, Sequence, Union

import numpy as np
import torch
from scipy.signal import lfilter as _lfilter64, residuez

from .. import _lib
from ._common import check_input, require_hip

__all__ = ["HipIIR", "parallel_sections", "sections_struct"]

#: largest realisation error (peak relative, impulse response in float64)
_REALISATION_TOL = 1e-9


def _as_coeffs(values) -> np.ndarray:
    if isinstance(values, torch.Tensor):
        values = values.detach().cpu().double().numpy()
    return np.asarray(values, dtype=np.float64).ravel()


def _impulse(sections, c0, taps):
    """Impulse response of a parallel form in float64."""

    x = np.zeros(taps)
    x[0] = 1.0
    y = c0 * x
    for b0, b1, b2, a1, a2 in sections:
        y = y + _lfilter64([b0, b1, b2], [1.0, a1, a2], x)
    return y


def parallel_sections(b_coeffs, a_coeffs, taps: int = 4096):
    """Parallel second order sections of ``b / a``.

    Returns ``(c0, [(b0, b1, b2, a1, a2), ...])`` with float64 values.
    """

    b, a = _as_coeffs(b_coeffs), _as_coeffs(a_coeffs)
    size = max(b.shape[0], a.shape[0])
    b = np.pad(b, (0, size - b.shape[0]))
    a = np.pad(a, (0, size - a.shape[0]))
    if a[0] == 0.0:
        raise ValueError("The leading denominator coefficient a[0] must not be zero.")
    b, a = b / a[0], a / a[0]

    # trailing zero denominator terms do not add poles
    order = size - 1
    while order > 0 and a[order] == 0.0:
        order -= 1
    if order < 1:
        raise ValueError("The HIP IIR filter needs at least one pole.")
    if np.any(b[order + 1 :] != 0.0):
        raise RuntimeError(
            "The numerator is longer than the denominator; such a filter has an FIR "
            "tail that the parallel realisation does not represent."
        )
    b, a = b[: order + 1], a[: order + 1]

    if order <= 2:
        bb = np.pad(b, (0, 3 - b.shape[0]))
        aa = np.pad(a, (0, 3 - a.shape[0]))
        return 0.0, [(bb[0], bb[1], bb[2], aa[1], aa[2])]

    r, p, k = residuez(b, a)
    if len(k) > 1:
        raise RuntimeError("Unexpected FIR terms in the partial fraction expansion.")
    c0 = float(k[0]) if len(k) else 0.0

    used = np.zeros(len(p), dtype=bool)
    complex_secs, reals = [], []
    for i in range(len(p)):
        if used[i]:
            continue
        used[i] = True
        if abs(p[i].imag) <= 1e-12 * max(1.0, abs(p[i])):
            reals.append((p[i].real, r[i].real))
            continue
        dist = np.where(used, np.inf, np.abs(p - np.conj(p[i])))
        j = int(np.argmin(dist))
        if not np.isfinite(dist[j]) or dist[j] > 1e-8 * max(1.0, abs(p[i])):
            raise RuntimeError("Could not pair a complex pole with its conjugate.")
        used[j] = True
        pr, rr = p[i], r[i]
        complex_secs.append(
            (2 * rr.real, -2 * (rr * np.conj(pr)).real, 0.0, -2 * pr.real, abs(pr) ** 2)
        )

    reals.sort(key=lambda v: -abs(v[0]))
    real_secs = []
    for idx in range(0, len(reals) - 1, 2):
        (p1, r1), (p2, r2) = reals[idx], reals[idx + 1]
        real_secs.append((r1 + r2, -(r1 * p2 + r2 * p1), 0.0, -(p1 + p2), p1 * p2))
    if len(reals) % 2:
        p1, r1 = reals[-1]
        real_secs.append((r1, 0.0, 0.0, -p1, 0.0))

    sections = real_secs + complex_secs
    # the first output sample is b0 x; choosing the direct term from it keeps
    # h[0] exact instead of a difference of large residues
    c0 = float(b[0]) - float(sum(sec[0] for sec in sections))
    if len(sections) > _lib.MAX_SECTIONS:
        raise RuntimeError(
            f"The filter needs {len(sections)} parallel sections, at most "
            f"{_lib.MAX_SECTIONS} are supported (order <= 16)."
        )

    reference = _lfilter64(b, a, np.eye(1, taps)[0])
    scale = max(float(np.abs(reference).max()), 1e-300)
    error = float(np.abs(_impulse(sections, c0, taps) - reference).max()) / scale
    if not math.isfinite(error) or error > _REALISATION_TOL:
        raise RuntimeError(
            f"The parallel realisation of this filter misses its impulse response by "
            f"{error:.3g} (peak relative); repeated or clustered poles cannot be realised "
            f"in parallel form. Split the filter into second order sections and chain "
            f"several HipIIR modules instead."
        )
    if np.any(np.abs(p) >= 1.0):
        warnings.warn(
            "The filter has poles on or outside the unit circle; its output grows "
            "without bound.",
            RuntimeWarning,
            stacklevel=3,
        )
    return c0, sections


def sections_struct(c0, sections) -> _lib.IirSections:
    """``pesq_iir_sections`` of a parallel form."""

    out = _lib.IirSections()
    out.count = len(sections)
    out.c0 = float(c0)
    for i, (b0, b1, b2, a1, a2) in enumerate(sections):
        out.b0[i], out.b1[i], out.b2[i] = float(b0), float(b1), float(b2)
        out.a1[i], out.a2[i] = float(a1), float(a2)
    return out


def _pack_table(struct: _lib.IirSections) -> torch.Tensor:
    lib = _lib.library()
    buf = (ctypes.c_ubyte * lib.pesq_iir_table_bytes())()
    _lib.check(lib.pesq_iir_table_pack(ctypes.byref(struct), buf), "pesq_iir_table_pack")
    return torch.frombuffer(bytearray(buf), dtype=torch.uint8).clone()


def _launch(signal: torch.Tensor, table: torch.Tensor, sections: int, reverse: bool):
    if table.device != signal.device:
        raise RuntimeError(
            f"The filter tables live on {table.device} but the signal on {signal.device}; "
            "move the module with `.to(signal.device)` first."
        )
    lib = _lib.library()
    rows, length = signal.shape
    out = torch.empty_like(signal)
    if rows == 0 or length == 0:
        return out
    ws_bytes = _lib.size_query(lib.pesq_iir_workspace, rows, length)
    workspace = torch.empty(max(ws_bytes, 8), dtype=torch.uint8, device=signal.device)
    with torch.cuda.device(signal.device):
        _lib.check(
            lib.pesq_iir_apply(
                _lib.ptr(signal),
                _lib.ptr(out),
                rows,
                length,
                _lib.ptr(table),
                sections,
                int(reverse),
                _lib.ptr(workspace),
                _lib.stream_handle(signal.device),
            ),
            "pesq_iir_apply",
        )
    return out


class _IIRFunction(torch.autograd.Function):
    """Forward filter; the backward is the same filter time reversed."""

    @staticmethod
    def forward(ctx, signal, table, sections, reverse):
        ctx.table, ctx.sections, ctx.reverse = table, sections, reverse
        return _launch(signal, table, sections, reverse)

    @staticmethod
    def backward(ctx, grad):
        grad = grad.contiguous()
        reverse = not ctx.reverse
        if torch.is_grad_enabled() and grad.requires_grad:
            out = _IIRFunction.apply(grad, ctx.table, ctx.sections, reverse)
        else:
            out = _launch(grad, ctx.table, ctx.sections, reverse)
        return out, None, None, None


class HipIIR(torch.nn.Module):
    """Causal IIR filter with zero initial conditions, evaluated on the GPU.

    Numerically ``torchaudio.functional.lfilter(x, a_coeffs, b_coeffs,
    clamp=False)`` evaluated with a float64 state, as a chunked parallel scan
    over the time axis.  Same constructor as ``TritonIIR``
    (``iir.py:1343-1375``); ``chunk_size`` and ``method`` are accepted for
    compatibility, the chunk geometry is fixed by the kernels.

    Attributes
    ----------
    order : int
        Number of poles of the difference equation
    sections : int
        Parallel second order sections of the realisation
    basis : str
        ``"parallel"`` (or ``"section"`` for a single biquad)
    """

    def __init__(
        self,
        b_coeffs: Union[Sequence[float], np.ndarray, torch.Tensor],
        a_coeffs: Union[Sequence[float], np.ndarray, torch.Tensor],
        chunk_size: Optional[Union[int, str]] = None,
        method: str = "auto",
    ):
        super().__init__()
        if method not in ("auto", "scan", "matmul"):
            raise ValueError(f"Unknown method `{method}`.")
        if chunk_size not in (None, "tune"):
            chunk_size = int(chunk_size)
            if chunk_size < 64 or chunk_size % 64 != 0:
                raise ValueError("`chunk_size` has to be a positive multiple of 64.")

        numerator, denominator = _as_coeffs(b_coeffs), _as_coeffs(a_coeffs)
        c0, sections = parallel_sections(numerator, denominator)
        self.order = max(numerator.shape[0], denominator.shape[0]) - 1
        self.sections = len(sections)
        self.basis = "section" if self.order <= 2 else "parallel"
        self.c0 = c0
        self.section_coeffs = sections
        self.register_buffer(
            "table", _pack_table(sections_struct(c0, sections)), persistent=False
        )

    def forward(self, signal: torch.Tensor) -> torch.Tensor:
        """Filter a ``[batch, sample]`` signal along the sample axis."""

        signal = check_input(signal, "signal")
        if signal.dim() != 2:
            raise RuntimeError(
                f"The HIP IIR filter needs a [batch, sample] tensor, got {tuple(signal.shape)}."
            )
        if signal.shape[1] == 0:
            return signal.clone()
        require_hip()
        if not (torch.is_grad_enabled() and signal.requires_grad):
            return _launch(signal, self.table, self.sections, False)
        return _IIRFunction.apply(signal, self.table, self.sections, False)
