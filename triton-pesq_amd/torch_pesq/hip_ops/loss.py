"""``PesqLossHip``: the drop-in for ``PesqLossTriton`` (``torch_pesq/triton_ops/loss.py:18-215``).

Same module as :class:`torch_pesq.loss.PesqLoss` plus :meth:`graphed`, which
captures forward and backward into HIP graphs for one input shape.
"""

import torch

from ..loss import PesqLoss

__all__ = ["PesqLossHip", "PesqLossTriton"]


class PesqLossHip(PesqLoss):
    """PESQ loss on HIP kernels with HIP graph capture."""

    def graphed(self, ref: torch.Tensor, deg: torch.Tensor):
        """Capture the loss in HIP graphs, specialised to one input shape.

        Mirrors ``triton_ops/loss.py:149-201``: detached sample copies with the
        same ``requires_grad`` flags and one warm-up on a side stream (nothing
        is tuned at run time here; the warm-up loads the kernels before the
        capture).  The returned callable replaces ``self.__call__`` for this
        shape and these flags and is bit exact with the eager path, loss and
        gradients.  As with the reference's ``make_graphed_callables``, the
        loss and the gradients it returns are static buffers that the next
        call overwrites.  Unlike the reference, ``self`` is left untouched, so
        the module keeps working for other shapes.

        At the PESQ geometry the graphs are captured by the C++ extension
        (``GraphedLoss``: the forward and backward library calls, and the
        resampler's when the rate is not 16 kHz), whose autograd node replays
        them with no Python in between.  Other STFT geometries, which run the
        per stage operators, go through ``torch.cuda.make_graphed_callables``.
        """

        sample = tuple(t.detach().clone().requires_grad_(t.requires_grad) for t in (ref, deg))
        target = _LossCall(self)
        stream = torch.cuda.Stream()
        stream.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(stream):
            output = target(*sample)
            if output.requires_grad:
                torch.autograd.grad(output.sum(), [t for t in sample if t.requires_grad])
        torch.cuda.current_stream().wait_stream(stream)
        torch.cuda.synchronize()
        if self.general:
            return torch.cuda.make_graphed_callables(target, sample)

        from .. import _lib

        return _lib.torch_ext().GraphedLoss(
            sample[0], sample[1], self.model_table, float(self.factor), *self._bank(sample[0])
        )

    def graphed_step(self, ref: torch.Tensor, deg: torch.Tensor):
        """``grad(self(ref, deg).sum(), inputs)`` as one HIP graph, for one input shape.

        Not in the reference, whose graphs stop at the autograd boundary: the
        forward and the backward (upstream gradients of one, the derivative
        of the sum) of the inputs whose examples require a gradient, captured
        together.  The returned object has ``inputs()`` (the static ``ref``,
        ``deg`` to write into), ``replay()`` (on the current stream) and
        ``outputs()`` (the static loss and the gradients of ``ref`` and
        ``deg``, ``None`` where not requested), all bit exact with the eager
        step.  The PESQ geometry only (the fused pipeline).
        """

        if self.general:
            raise ValueError("graphed_step needs the PESQ geometry (the fused pipeline).")
        if not (ref.requires_grad or deg.requires_grad):
            raise ValueError("graphed_step: ref or deg must require a gradient.")
        sample = tuple(t.detach().clone().requires_grad_(t.requires_grad) for t in (ref, deg))
        stream = torch.cuda.Stream()
        stream.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(stream):
            output = self(*sample)
            torch.autograd.grad(output.sum(), [t for t in sample if t.requires_grad])
        torch.cuda.current_stream().wait_stream(stream)
        torch.cuda.synchronize()

        from .. import _lib

        step = _lib.torch_ext().GraphedStep(
            sample[0], sample[1], self.model_table, float(self.factor), *self._bank(sample[0])
        )
        static_ref, static_deg = step.inputs()
        with torch.no_grad():
            static_ref.copy_(ref)
            static_deg.copy_(deg)
        return step

    def _bank(self, example: torch.Tensor):
        """The resampler's tables and sizes for the graphed classes (empty at 16 kHz)."""

        rs = self.resampler
        if rs.orig_freq == rs.new_freq:
            return [], []
        bank, steps = rs.bank()
        return bank, steps + [rs.output_length(example.shape[-1])]


class _LossCall(torch.nn.Module):
    """``loss(ref, deg)`` of a :class:`PesqLossHip` as a capturable module."""

    def __init__(self, loss: PesqLossHip):
        super().__init__()
        # a plain attribute, not a submodule: the capture must not see (and
        # re-register) the loss module's constant parameters
        object.__setattr__(self, "loss", loss)

    def forward(self, ref: torch.Tensor, deg: torch.Tensor) -> torch.Tensor:
        return self.loss(ref, deg)


#: the reference's name for the GPU backend class
PesqLossTriton = PesqLossHip
