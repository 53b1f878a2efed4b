"""HIP polyphase resampler, the ``TritonResample`` operator (``resample.py:442-574``).

Same constructor and attributes as the reference (``kernel``, ``kernel_t``
is not needed, ``width``, ``orig_step``, ``new_step``).  Forward and adjoint
are HIP kernels (``csrc/resample.hip``) that evaluate only the non-zero taps
of each phase.  The autograd nodes are C++ (``csrc/torch_autograd.cpp``):
the adjoint is itself differentiable (its derivative is the forward), which
gives a working double backward like the reference's ``_ResampleAdjoint``
(``resample.py:381-410``).
"""

import ctypes
import math
from typing import Optional

import torch

from .. import _lib
from ._common import check_input
from .sinc import resample_length, sinc_resample_kernel

__all__ = ["HipResample", "resample_launch"]

_INDEX_LIMIT = 2**31 - 1


def resample_launch(src: torch.Tensor, n_other: int, module: "HipResample", forward: bool):
    """One forward (``[rows, n_in] -> [rows, n_other]``) or adjoint
    (``[rows, n_out] -> [rows, n_other]``) launch, outside autograd.

    The same library calls the C++ autograd nodes make; used to time the
    kernels alone.
    """

    lib = _lib.library()
    rows = src.shape[0]
    n_in, n_out = (src.shape[1], n_other) if forward else (n_other, src.shape[1])
    out = torch.empty((rows, n_other), dtype=torch.float32, device=src.device)
    info = module.plan_info
    with torch.cuda.device(src.device):
        if (info.fwd_span if forward else info.bwd_span) > 0:
            name = "pesq_resample_plan_forward" if forward else "pesq_resample_plan_backward"
            _lib.check(
                getattr(lib, name)(
                    _lib.ptr(src), _lib.ptr(out), rows, n_in, n_out, ctypes.byref(info),
                    _lib.ptr(module.plan), _lib.stream_handle(src.device),
                ),
                name,
            )
            return out
        name = "pesq_resample_forward" if forward else "pesq_resample_backward"
        lo, hi = (module.tap_lo, module.tap_hi) if forward else (module.phase_lo, module.phase_hi)
        _lib.check(
            getattr(lib, name)(
                _lib.ptr(src), _lib.ptr(out), rows, n_in, n_out, _lib.ptr(module.kernel),
                _lib.ptr(lo), _lib.ptr(hi), module.orig_step, module.new_step, module.width,
                module.kernel.shape[1], _lib.stream_handle(src.device),
            ),
            name,
        )
    return out


class HipResample(torch.nn.Module):
    """Resample a signal from one rate to another with HIP kernels.

    Numerically ``torchaudio.transforms.Resample`` with the same arguments,
    with float64 accumulation of the taps.  Identity (no kernel launch, any
    device) when both rates are equal.
    """

    def __init__(
        self,
        orig_freq: int = 16000,
        new_freq: int = 16000,
        lowpass_filter_width: int = 6,
        rolloff: float = 0.99,
        resampling_method: str = "sinc_interp_hann",
        beta: Optional[float] = None,
    ):
        super().__init__()
        if orig_freq <= 0 or new_freq <= 0:
            raise ValueError("Original and desired frequency have to be positive.")
        self.orig_freq, self.new_freq = int(orig_freq), int(new_freq)
        self.gcd = math.gcd(self.orig_freq, self.new_freq)
        self.orig_step = self.orig_freq // self.gcd
        self.new_step = self.new_freq // self.gcd
        self.lowpass_filter_width = lowpass_filter_width
        self.rolloff = rolloff
        self.resampling_method = resampling_method
        self.beta = beta
        self._lengths = {}  # output length per input length

        if self.orig_freq == self.new_freq:
            self.width = 0
            return

        kernel, self.width = sinc_resample_kernel(
            self.orig_freq, self.new_freq, lowpass_filter_width, rolloff, resampling_method, beta
        )
        nonzero = kernel != 0
        ntaps = kernel.shape[1]
        tap_lo = torch.zeros(self.new_step, dtype=torch.int32)
        tap_hi = torch.zeros(self.new_step, dtype=torch.int32)
        for j in range(self.new_step):
            idx = torch.nonzero(nonzero[j]).flatten()
            if idx.numel():
                tap_lo[j], tap_hi[j] = int(idx[0]), int(idx[-1]) + 1
        phase_lo = torch.zeros(ntaps, dtype=torch.int32)
        phase_hi = torch.zeros(ntaps, dtype=torch.int32)
        for k in range(ntaps):
            # phases whose non-zero band [tap_lo, tap_hi) contains k
            inside = torch.nonzero((tap_lo <= k) & (k < tap_hi)).flatten()
            if inside.numel():
                phase_lo[k], phase_hi[k] = int(inside[0]), int(inside[-1]) + 1
                span = torch.arange(int(phase_lo[k]), int(phase_hi[k]))
                assert bool(((tap_lo[span] <= k) & (k < tap_hi[span])).all()), "bands not monotone"
        self.register_buffer("kernel", kernel.contiguous())
        self.register_buffer("tap_lo", tap_lo)
        self.register_buffer("tap_hi", tap_hi)
        self.register_buffer("phase_lo", phase_lo)
        self.register_buffer("phase_hi", phase_hi)
        # compact tap tables of the tiled kernels (csrc/resample.hip)
        lib = _lib.library()
        info = _lib.ResamplePlanInfo()
        bank = kernel.contiguous()
        args = (bank.data_ptr(), tap_lo.data_ptr(), tap_hi.data_ptr(),
                self.orig_step, self.new_step, self.width, ntaps)
        _lib.check(lib.pesq_resample_plan(*args, ctypes.byref(info), None), "pesq_resample_plan")
        plan = torch.zeros(max(int(info.bytes), 4), dtype=torch.uint8)
        _lib.check(lib.pesq_resample_plan(*args, ctypes.byref(info), plan.data_ptr()),
                   "pesq_resample_plan")
        self.plan_info = info
        # host copy of the geometry for the C++ autograd nodes (stays on the CPU)
        self.plan_bytes = torch.frombuffer(bytearray(bytes(info)), dtype=torch.uint8)
        self.register_buffer("plan", plan)

    def output_length(self, n_samples: int) -> int:
        n = self._lengths.get(n_samples)
        if n is None:
            n = self._lengths[n_samples] = resample_length(n_samples, self.orig_step, self.new_step)
        return n

    def check_length(self, n_in: int, n_out: int) -> None:
        """Raise when a row of n_in samples (n_out out) exceeds the 32 bit launch grid."""

        slack = 128 * max(self.orig_step, self.new_step) + self.kernel.shape[1]
        if max(n_in, n_out) > _INDEX_LIMIT - slack:
            raise RuntimeError("The signal is too long for the resampler's 32 bit launch grid.")

    def bank(self):
        """The filter tables and steps the C++ entry points take, ``(tensors, steps)``."""

        return (
            [self.kernel, self.tap_lo, self.tap_hi, self.phase_lo, self.phase_hi, self.plan,
             self.plan_bytes],
            [self.orig_step, self.new_step, self.width],
        )

    def forward(self, waveform: torch.Tensor) -> torch.Tensor:
        """Resample ``[..., sample]`` signals along the last axis."""

        if self.orig_freq == self.new_freq:
            return waveform
        if self.kernel.device != waveform.device:
            raise RuntimeError(
                f"The resampling kernel lives on {self.kernel.device} but the waveform on "
                f"{waveform.device}, move the module with `.to(...)`."
            )
        shape = waveform.shape
        batch = math.prod(shape[:-1])
        packed = check_input(waveform.reshape(batch, shape[-1]), "waveform")
        n_out = self.output_length(shape[-1])
        self.check_length(shape[-1], n_out)
        out = _lib.torch_ext().resample(
            packed, n_out, self.kernel, self.tap_lo, self.tap_hi, self.phase_lo, self.phase_hi,
            self.plan, self.plan_bytes, self.orig_step, self.new_step, self.width,
        )
        return out.reshape(shape[:-1] + out.shape[-1:])

    def extra_repr(self) -> str:
        return f"orig_freq={self.orig_freq}, new_freq={self.new_freq}"
