"""Element-wise stages as HIP operators (``torch_pesq/triton_ops/elementwise.py``).

``peak_normalize``, ``edge_ramp``, ``align_scale`` and ``pesq_epilogue`` keep
the reference's signatures, semantics and gradient conventions:

* ``peak_normalize``: the common peak is a constant in the backward
  (exact for the composed pipeline by scale invariance,
  ``elementwise.py:165-176``); IEEE division, bit exact with ``x / peak``;
* ``edge_ramp``: ``(x * head) * tail`` in float32, bit exact, its own adjoint;
* ``align_scale``: reductions in float64 (two fixed-order stages);
* ``pesq_epilogue``: MOS and loss, gradients for either or both.
"""

import torch

from .. import _lib
from ._common import check_input

__all__ = ["peak_normalize", "edge_ramp", "align_scale", "pesq_epilogue"]

_MAX_ROW = 2**31 - 4096


def _workspace(rows, device):
    lib = _lib.library()
    size = _lib.size_query(lib.pesq_elementwise_workspace, rows)
    return torch.empty(max(size, 8), dtype=torch.uint8, device=device)


def _call(name, *args, device):
    lib = _lib.library()
    with torch.cuda.device(device):
        _lib.check(getattr(lib, name)(*args, _lib.stream_handle(device)), name)


class _PeakNormalize(torch.autograd.Function):
    @staticmethod
    def forward(ctx, ref, deg, stack=False):
        ref, deg = check_input(ref, "ref"), check_input(deg, "deg")
        if ref.ndim != 2 or deg.ndim != 2:
            raise RuntimeError(
                f"peak_normalize expects [batch, sample] tensors, got {tuple(ref.shape)} and {tuple(deg.shape)}."
            )
        if ref.shape != deg.shape:
            raise RuntimeError(
                f"peak_normalize expects matching shapes, got {tuple(ref.shape)} and {tuple(deg.shape)}."
            )
        batch, n = ref.shape
        if n == 0:
            raise RuntimeError("peak_normalize needs at least one sample.")
        if n > _MAX_ROW:
            raise RuntimeError(f"peak_normalize supports at most {_MAX_ROW} samples per row, got {n}.")
        peak = torch.empty(batch, device=ref.device)
        if stack:
            stacked = torch.empty((2 * batch, n), device=ref.device)
            out_ref, out_deg = stacked[:batch], stacked[batch:]
        else:
            out_ref, out_deg = torch.empty_like(ref), torch.empty_like(deg)
        ws = _workspace(batch, ref.device)
        _call("pesq_peak_normalize_forward", _lib.ptr(ref), _lib.ptr(deg), batch, n,
              _lib.ptr(out_ref), _lib.ptr(out_deg), _lib.ptr(peak), _lib.ptr(ws), device=ref.device)
        ctx.save_for_backward(peak)
        ctx.shape, ctx.stack = (batch, n), stack
        return stacked if stack else (out_ref, out_deg)

    @staticmethod
    def backward(ctx, *grads):
        (peak,) = ctx.saved_tensors
        batch, n = ctx.shape
        need_ref, need_deg = ctx.needs_input_grad[:2]
        if not need_ref and not need_deg:
            return None, None, None
        if ctx.stack:
            g = check_input(grads[0], "grad")
            g_ref, g_deg = g[:batch], g[batch:]
        else:
            g_ref = check_input(grads[0], "grad_ref") if grads[0] is not None else torch.zeros(batch, n, device=peak.device)
            g_deg = check_input(grads[1], "grad_deg") if grads[1] is not None else torch.zeros(batch, n, device=peak.device)
        out_ref = torch.empty((batch, n), device=peak.device) if need_ref else None
        out_deg = torch.empty((batch, n), device=peak.device) if need_deg else None
        _call("pesq_peak_normalize_backward", _lib.ptr(g_ref if need_ref else None),
              _lib.ptr(g_deg if need_deg else None), _lib.ptr(peak), batch, n,
              _lib.ptr(out_ref), _lib.ptr(out_deg), device=peak.device)
        return out_ref, out_deg, None


def peak_normalize(ref, deg, stack=False):
    """Divide both signals by their common peak (``elementwise.py:272-300``)."""

    return _PeakNormalize.apply(ref, deg, stack)


class _EdgeRamp(torch.autograd.Function):
    @staticmethod
    def forward(ctx, x):
        x = check_input(x, "x")
        if x.ndim != 2:
            raise RuntimeError(f"edge_ramp expects a [batch, sample] tensor, got {tuple(x.shape)}.")
        rows, n = x.shape
        if n < 15:
            raise RuntimeError(
                f"edge_ramp needs at least 15 samples, the length of a single ramp, got {n}."
            )
        out = torch.empty_like(x)
        _call("pesq_edge_ramp", _lib.ptr(x), _lib.ptr(out), rows, n, device=x.device)
        return out

    @staticmethod
    def backward(ctx, grad):
        if not ctx.needs_input_grad[0]:
            return None
        grad = check_input(grad, "grad_out")
        out = torch.empty_like(grad)
        _call("pesq_edge_ramp", _lib.ptr(grad), _lib.ptr(out), grad.shape[0], grad.shape[1],
              device=grad.device)
        return out


def edge_ramp(x):
    """Fade the first and last 15 samples (``elementwise.py:389-408``)."""

    return _EdgeRamp.apply(x)


class _AlignScale(torch.autograd.Function):
    @staticmethod
    def forward(ctx, signal, filtered):
        signal, filtered = check_input(signal, "signal"), check_input(filtered, "filtered")
        if signal.ndim != 2 or filtered.ndim != 2:
            raise RuntimeError(
                f"align_scale expects [batch, sample] tensors, got {tuple(signal.shape)} and {tuple(filtered.shape)}."
            )
        if signal.shape[0] != filtered.shape[0]:
            raise RuntimeError(
                f"align_scale expects a matching batch size, got {signal.shape[0]} and {filtered.shape[0]}."
            )
        rows, n_sig = signal.shape
        n_flt = filtered.shape[1]
        if n_sig == 0 or n_flt == 0:
            raise RuntimeError("align_scale needs at least one sample.")
        out = torch.empty_like(signal)
        state = torch.empty((rows, 2), dtype=torch.float64, device=signal.device)
        ws = _workspace(rows, signal.device)
        _call("pesq_align_scale_forward", _lib.ptr(signal), _lib.ptr(filtered), rows, n_sig, n_flt,
              _lib.ptr(out), _lib.ptr(state), _lib.ptr(ws), device=signal.device)
        ctx.save_for_backward(signal, filtered, state)
        return out

    @staticmethod
    def backward(ctx, grad):
        signal, filtered, state = ctx.saved_tensors
        need_sig, need_flt = ctx.needs_input_grad[:2]
        if not need_sig and not need_flt:
            return None, None
        grad = check_input(grad, "grad_out")
        rows, n_sig = signal.shape
        n_flt = filtered.shape[1]
        g_sig = torch.empty_like(signal) if need_sig else None
        g_flt = torch.empty_like(filtered) if need_flt else None
        ws = _workspace(rows, signal.device)
        _call("pesq_align_scale_backward", _lib.ptr(grad), _lib.ptr(signal), _lib.ptr(filtered),
              _lib.ptr(state), rows, n_sig, n_flt, _lib.ptr(g_sig), _lib.ptr(g_flt), _lib.ptr(ws),
              device=signal.device)
        return g_sig, g_flt


def align_scale(signal, filtered):
    """Scale ``signal`` so the power of ``filtered`` is ``1e7`` (``elementwise.py:655-675``)."""

    return _AlignScale.apply(signal, filtered)


class _PesqEpilogue(torch.autograd.Function):
    @staticmethod
    def forward(ctx, d_symm, d_asymm, factor):
        d_symm, d_asymm = check_input(d_symm, "d_symm"), check_input(d_asymm, "d_asymm")
        if d_symm.ndim != 1 or d_asymm.ndim != 1:
            raise RuntimeError(
                f"pesq_epilogue expects [batch] tensors, got {tuple(d_symm.shape)} and {tuple(d_asymm.shape)}."
            )
        if d_symm.shape != d_asymm.shape:
            raise RuntimeError(
                f"pesq_epilogue expects matching shapes, got {tuple(d_symm.shape)} and {tuple(d_asymm.shape)}."
            )
        if isinstance(factor, torch.Tensor) and factor.requires_grad:
            raise RuntimeError(
                "pesq_epilogue treats `factor` as a constant, pass a Python float. A tensor that "
                "requires a gradient would receive none."
            )
        mos, loss = torch.empty_like(d_symm), torch.empty_like(d_symm)
        _call("pesq_epilogue_forward", _lib.ptr(d_symm), _lib.ptr(d_asymm), d_symm.shape[0],
              float(factor), _lib.ptr(mos), _lib.ptr(loss), device=d_symm.device)
        ctx.save_for_backward(d_symm, d_asymm)
        ctx.factor = float(factor)
        ctx.set_materialize_grads(False)
        return mos, loss

    @staticmethod
    def backward(ctx, g_mos, g_loss):
        d_symm, d_asymm = ctx.saved_tensors
        need_ds, need_da = ctx.needs_input_grad[:2]
        if (not need_ds and not need_da) or (g_mos is None and g_loss is None):
            return None, None, None
        g_mos = check_input(g_mos, "grad_mos") if g_mos is not None else None
        g_loss = check_input(g_loss, "grad_loss") if g_loss is not None else None
        g_ds, g_da = torch.empty_like(d_symm), torch.empty_like(d_asymm)
        _call("pesq_epilogue_backward", _lib.ptr(d_symm), _lib.ptr(d_asymm), _lib.ptr(g_mos),
              _lib.ptr(g_loss), d_symm.shape[0], ctx.factor, _lib.ptr(g_ds), _lib.ptr(g_da),
              device=d_symm.device)
        return (g_ds if need_ds else None), (g_da if need_da else None), None


def pesq_epilogue(d_symm, d_asymm, factor):
    """``(mos, loss)`` from the two distances (``elementwise.py:835-854``)."""

    return _PesqEpilogue.apply(d_symm, d_asymm, factor)
