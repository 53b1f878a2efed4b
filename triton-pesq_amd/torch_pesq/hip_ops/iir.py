"""HIP IIR filter, the ``TritonIIR`` operator (``torch_pesq/triton_ops/iir.py:1266-1482``).

Realisations
------------
Every section is a direct form II transposed biquad with a float64 state,
scanned over the time axis in chunks (``csrc/iir.hpp``).  Two realisations of
a difference equation ``b / a`` are built on the host and scored by how well
their float64 impulse response reproduces the one of the difference equation
itself (``scipy.signal.lfilter`` in float64), the *fidelity*:

``parallel``
    the partial fraction expansion (``scipy.signal.residuez``): a direct term
    ``c0`` and one residue per pole; conjugate pole pairs, and pairs of real
    poles, merged into second order sections,
    ``H(z) = c0 + sum_k (b0_k + b1_k z^-1) / (1 + a1_k z^-1 + a2_k z^-2)``.
    The sections are independent, so all of them run in one scan pass.  It
    does not exist for repeated poles and loses digits for clustered ones.
``cascade``
    the series of biquads of ``scipy.signal.tf2sos``, one scan pass per
    section with float64 signals between the passes.  It handles repeated
    poles, zero poles and numerators longer than the denominator.

The parallel form is used whenever its fidelity is within 1e-9 (one pass
instead of one per section), otherwise the realisation with the better
fidelity.  Order <= 2 filters are a single full biquad.  The score is rated
with the reference's limits (``iir.py:38-58``, :func:`_state_space`
``iir.py:599-666``): above ``1e5 * 2^-24`` the filter is rejected with a
``RuntimeError`` (its result would carry no significant digit), above
``1e3 * 2^-24`` it warns that the accuracy is degraded.  With the float64
state the runtime conditioning term of the reference's score (table entries
times the float32 unit round off) does not apply; what remains is the
fidelity of the realisation, which is what separates the orders that the
reference accepts (16), flags (20) and rejects (30).

Backward
--------
The filter is a lower triangular Toeplitz operator T, so its adjoint is
J T J (J = time reversal): the same filter run over the reversed signal.  The
kernels do the reversal by index, like the reference (``iir.py:1232-1258``);
in the cascade every pass is reversed, J T_K J ... J T_1 J = J T J.
"""

import ctypes
import math
import warnings
from typing import NamedTuple, Optional, Sequence, Union

import numpy as np
import torch
from scipy.signal import lfilter as _lfilter64, residuez, sosfilt, tf2sos

from .. import _lib
from ._common import check_input, require_hip

__all__ = ["HipIIR", "Realisation", "realise", "parallel_sections", "sections_struct"]

#: largest realisation error (peak relative, impulse response in float64) of
#: the parallel form used by the PESQ pipeline, and below which the stand-alone
#: filter prefers it
_REALISATION_TOL = 1e-9

#: the reference's rating of a realisation's predicted peak relative error
#: (``iir.py:38-58``): rejected above the first, flagged above the second
_ERROR_LIMIT = 1e5 * 2.0**-24
_ERROR_WARN = 1e3 * 2.0**-24

#: impulse response horizon the realisations are scored over
_SCORE_TAPS = 4096


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


def _parallel_form(b_coeffs, a_coeffs):
    """Parallel second order sections of ``b / a``, without the fidelity check.

    Returns ``(b, a, c0, [(b0, b1, b2, a1, a2), ...])``: the normalised and
    trimmed coefficients and the float64 realisation.  Raises ``RuntimeError``
    when the filter has no parallel form of at most ``MAX_SECTIONS`` sections.
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
        return b, a, 0.0, [(bb[0], bb[1], bb[2], aa[1], aa[2])]

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
    return b, a, c0, sections


def _unstable_warning(a) -> None:
    if np.any(np.abs(np.roots(a)) >= 1.0):
        warnings.warn(
            "The filter has poles on or outside the unit circle; its output grows "
            "without bound.",
            RuntimeWarning,
            stacklevel=4,
        )


def parallel_sections(b_coeffs, a_coeffs, taps: int = 4096):
    """Parallel second order sections of ``b / a``, validated to 1e-9.

    Returns ``(c0, [(b0, b1, b2, a1, a2), ...])`` with float64 values; raises
    ``RuntimeError`` when the parallel form misses the float64 impulse
    response of the difference equation by more than 1e-9 (peak relative).
    """

    b, a, c0, sections = _parallel_form(b_coeffs, a_coeffs)
    if len(sections) == 1 and a.shape[0] <= 3:
        return c0, sections
    reference = _lfilter64(b, a, np.eye(1, taps)[0])
    scale = max(float(np.abs(reference).max()), 1e-300)
    error = float(np.abs(_impulse(sections, c0, taps) - reference).max()) / scale
    if not math.isfinite(error) or error > _REALISATION_TOL:
        raise RuntimeError(
            f"The parallel realisation of this filter misses its impulse response by "
            f"{error:.3g} (peak relative); repeated or clustered poles cannot be realised "
            f"in parallel form."
        )
    _unstable_warning(a)
    return c0, sections


class Realisation(NamedTuple):
    """A realisation of a difference equation chosen by :func:`realise`.

    ``basis`` is ``"parallel"`` (``c0`` and ``(b0, b1, b2, a1, a2)`` rows) or
    ``"cascade"`` (``sos`` rows ``(b0, b1, b2, a0, a1, a2)``); ``score`` is the
    peak relative error of its float64 impulse response against the one of
    the difference equation.
    """

    basis: str
    c0: float
    sections: np.ndarray
    score: float
    order: int


def _normalised(b_coeffs, a_coeffs):
    """``b``, ``a`` padded to one length and divided by ``a[0]`` (``iir.py:187-214``)."""

    b, a = _as_coeffs(b_coeffs), _as_coeffs(a_coeffs)
    size = max(b.shape[0], a.shape[0])
    if a.shape[0] == 0 or a[0] == 0.0:
        raise ValueError("The leading denominator coefficient a[0] must not be zero.")
    b = np.pad(b, (0, size - b.shape[0]))
    a = np.pad(a, (0, size - a.shape[0]))
    if size - 1 < 1:
        raise ValueError("The HIP IIR filter needs at least one pole.")
    return b / a[0], a / a[0]


def _fidelity(response, reference, scale) -> float:
    with np.errstate(all="ignore"):
        error = float(np.abs(response - reference).max()) / scale
    return error if math.isfinite(error) else math.inf


def realise(b_coeffs, a_coeffs, taps: int = _SCORE_TAPS) -> Realisation:
    """The realisation the HIP filter runs for ``b / a``.

    Builds the parallel form and the cascade, scores both by the fidelity of
    their float64 impulse response over ``taps`` samples, prefers the
    parallel form when it is within 1e-9, else takes the better one, and rates
    the result like the reference's ``_state_space`` (``iir.py:599-666``):
    ``RuntimeError`` above ``1e5 * 2^-24``, a ``RuntimeWarning`` above
    ``1e3 * 2^-24``.
    """

    b, a = _normalised(b_coeffs, a_coeffs)
    order = b.shape[0] - 1
    impulse = np.eye(1, taps)[0]
    with np.errstate(all="ignore"):
        reference = _lfilter64(b, a, impulse)
    scale = max(float(np.abs(reference).max()), 1e-30)
    if not math.isfinite(scale):
        raise RuntimeError(
            "The impulse response of this filter overflows float64; no realisation of it "
            "carries significant digits."
        )

    candidates = []
    if order <= 2:
        bb, aa = np.pad(b, (0, 3 - b.shape[0])), np.pad(a, (0, 3 - a.shape[0]))
        sos = np.array([[bb[0], bb[1], bb[2], 1.0, aa[1], aa[2]]])
        candidates.append(("cascade", 0.0, sos, 0.0))
    else:
        try:
            _, _, c0, sections = _parallel_form(b, a)
            score = _fidelity(_impulse(sections, c0, taps), reference, scale)
            candidates.append(("parallel", c0, np.asarray(sections, dtype=np.float64), score))
        except (RuntimeError, ValueError, np.linalg.LinAlgError):
            pass
        try:
            with warnings.catch_warnings():
                warnings.simplefilter("ignore")
                sos = np.asarray(tf2sos(b, a), dtype=np.float64)
            if sos.shape[0] <= _lib.MAX_CASCADE:
                with np.errstate(all="ignore"):
                    response = sosfilt(sos, impulse)
                candidates.append(("cascade", 0.0, sos, _fidelity(response, reference, scale)))
        except (ValueError, np.linalg.LinAlgError):
            pass

    parallel = [c for c in candidates if c[0] == "parallel" and c[3] <= _REALISATION_TOL]
    best = parallel[0] if parallel else min(candidates, key=lambda c: c[3], default=None)
    if best is None or not math.isfinite(best[3]):
        raise RuntimeError(
            "Could not build a numerically valid realisation of the given coefficients."
        )
    name, c0, sections, score = best
    if score > _ERROR_LIMIT:
        raise RuntimeError(
            f"The best realisation of this filter (`{name}`, order {order}) misses the "
            f"impulse response of its difference equation by {score:.3g} (peak relative) "
            f"already in float64, so the result would carry no significant digits. Split "
            f"the filter into second order sections and chain several `HipIIR` modules "
            f"instead."
        )
    if score > _ERROR_WARN:
        warnings.warn(
            f"The realisation of this filter (`{name}`, order {order}) reproduces its "
            f"difference equation only to a peak relative error of about {score:.3g}; "
            f"accuracy will be degraded accordingly.",
            RuntimeWarning,
            stacklevel=3,
        )
    _unstable_warning(a)
    return Realisation(name, float(c0), sections, float(score), order)


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


def _pack_cascade(sos: np.ndarray) -> torch.Tensor:
    lib = _lib.library()
    rows = np.ascontiguousarray(sos, dtype=np.float64)
    buf = (ctypes.c_ubyte * (lib.pesq_iir_table_bytes() * rows.shape[0]))()
    _lib.check(
        lib.pesq_iir_cascade_pack(rows.ctypes.data_as(ctypes.c_void_p), rows.shape[0], buf),
        "pesq_iir_cascade_pack",
    )
    return torch.frombuffer(bytearray(buf), dtype=torch.uint8).clone()


def _launch(signal: torch.Tensor, table: torch.Tensor, basis: str, sections: int, reverse: bool):
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
    if basis == "cascade":
        ws_bytes = _lib.size_query(lib.pesq_iir_cascade_workspace, rows, length, sections)
        apply, name = lib.pesq_iir_cascade_apply, "pesq_iir_cascade_apply"
    else:
        ws_bytes = _lib.size_query(lib.pesq_iir_workspace, rows, length)
        apply, name = lib.pesq_iir_apply, "pesq_iir_apply"
    workspace = torch.empty(max(ws_bytes, 8), dtype=torch.uint8, device=signal.device)
    with torch.cuda.device(signal.device):
        _lib.check(
            apply(
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
            name,
        )
    return out


class _IIRFunction(torch.autograd.Function):
    """Forward filter; the backward is the same filter time reversed."""

    @staticmethod
    def forward(ctx, signal, table, basis, sections, reverse):
        ctx.table, ctx.basis, ctx.sections, ctx.reverse = table, basis, sections, reverse
        return _launch(signal, table, basis, sections, reverse)

    @staticmethod
    def backward(ctx, grad):
        grad = grad.contiguous()
        reverse = not ctx.reverse
        if torch.is_grad_enabled() and grad.requires_grad:
            out = _IIRFunction.apply(grad, ctx.table, ctx.basis, ctx.sections, reverse)
        else:
            out = _launch(grad, ctx.table, ctx.basis, ctx.sections, reverse)
        return out, None, None, None, None


class HipIIR(torch.nn.Module):
    """Causal IIR filter with zero initial conditions, evaluated on the GPU.

    Numerically ``torchaudio.functional.lfilter(x, a_coeffs, b_coeffs,
    clamp=False)`` evaluated with a float64 state, as a chunked parallel scan
    over the time axis.  Same constructor as ``TritonIIR``
    (``iir.py:1343-1375``); ``chunk_size`` is validated like there and
    ``method`` accepted, but the chunk geometry is fixed by the kernels (16
    samples per lane, 1024 per wavefront), so results do not depend on them.

    Attributes
    ----------
    order : int
        ``max(len(b), len(a)) - 1``, as in the reference
    basis : str
        ``"parallel"`` or ``"cascade"`` (see :func:`realise`)
    sections : int
        Second order sections of the realisation
    states : int
        Size of the state vector, two per section
    padded : int
        Same as ``states`` (the tables are not padded)
    score : float
        Peak relative error of the realisation's float64 impulse response
    candidates : tuple
        The chunk sizes the constructor was given (``TritonIIR.candidates``)

    Raises
    ------
    RuntimeError
        When no realisation reproduces the difference equation (see
        :func:`realise`); a degraded one warns.
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
            raise ValueError(f"Unknown method `{method}`, pick one of ('scan', 'matmul').")
        if chunk_size == "tune":
            candidates = (64, 128, 256, 512)
        elif chunk_size is None:
            candidates = (256,)
        else:
            chunk_size = int(chunk_size)
            if chunk_size < 64 or chunk_size % 64 != 0:
                raise ValueError("`chunk_size` has to be a positive multiple of 64.")
            candidates = (chunk_size,)
        self.method = "scan" if method == "auto" else method
        self.candidates = candidates

        numerator, denominator = _as_coeffs(b_coeffs), _as_coeffs(a_coeffs)
        real = realise(numerator, denominator)
        self.order = real.order
        self.basis = real.basis
        self.score = real.score
        self.sections = int(real.sections.shape[0])
        self.states = 2 * self.sections
        self.padded = self.states
        self.c0 = real.c0
        self.section_coeffs = real.sections
        if real.basis == "parallel":
            table = _pack_table(sections_struct(real.c0, real.sections))
        else:
            table = _pack_cascade(real.sections)
        self.register_buffer("table", table, persistent=False)

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
            return _launch(signal, self.table, self.basis, self.sections, False)
        return _IIRFunction.apply(signal, self.table, self.basis, self.sections, False)
