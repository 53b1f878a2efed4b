"""Float32 CPU restatement of the reference ``PesqLoss`` -- the CPU baseline.

TEST INFRASTRUCTURE ONLY (timed by ``bench.py``'s ``cpu_baseline`` leg and
exercised by ``tests/``; the shipped package never imports it).

It evaluates ``torch_pesq/loss.py:172-322`` with the same precision mix as
the reference running on CPU:

* float32 signal path: peak normalisation, ``lfilter`` (torchaudio's direct
  form I in float32: FIR part, then the all-pole recursion, oldest tap first,
  ``oracle/lfilter.c``), power alignment, ramp, ``torch.stft`` in float32;
* the Bark/loudness tables are float64 buffers in the reference
  (``bark.py:134-145``, ``loudness.py:44-55``), so from the Bark sums on the
  chain runs in float64, as it does there.

torchaudio's own float32 rounding is not reproducible without torchaudio
(absent here), so this is a baseline for timing and a second opinion on
accuracy, not a parity oracle.
"""

import ctypes
from pathlib import Path

import numpy as np
import torch

from . import pesq_oracle as O

_LIB = None


def _lib():
    global _LIB
    if _LIB is None:
        path = Path(__file__).with_name("liboracle.so")
        if not path.exists():
            from . import build

            build.build()
        lib = ctypes.CDLL(str(path))
        lib.lfilter_df1_f32.argtypes = [
            ctypes.c_void_p,
            ctypes.c_void_p,
            ctypes.c_int64,
            ctypes.c_int64,
            ctypes.c_void_p,
            ctypes.c_void_p,
            ctypes.c_int64,
            ctypes.c_int,
        ]
        lib.lfilter_df1_f32.restype = None
        _LIB = lib
    return _LIB


def lfilter_f32(x: torch.Tensor, b: torch.Tensor, a: torch.Tensor, reverse=False) -> torch.Tensor:
    x = x.detach().contiguous().float()
    b = b.detach().contiguous().float()
    a = a.detach().contiguous().float()
    y = torch.empty_like(x)
    _lib().lfilter_df1_f32(
        x.data_ptr(), y.data_ptr(), x.shape[0], x.shape[1], b.data_ptr(), a.data_ptr(), b.numel(), int(reverse)
    )
    return y


class _LFilter32(torch.autograd.Function):
    @staticmethod
    def forward(ctx, x, b, a):
        ctx.b, ctx.a = b, a
        return lfilter_f32(x, b, a)

    @staticmethod
    def backward(ctx, grad):
        return lfilter_f32(grad, ctx.b, ctx.a, reverse=True), None, None


def constants32():
    c = O.constants()
    return {
        "power_b": c["power_b"].float(),
        "power_a": c["power_a"].float(),
        "pre_b": c["pre_b"].float(),
        "pre_a": c["pre_a"].float(),
        "window": torch.hann_window(512),
        "fbank": c["fbank"].float(),
        "corr": c["corr"],  # float64 buffer in the reference
        "threshs": c["threshs"],  # float64
        "exp": c["exp"].float(),  # float32
        "width_bark": c["width_bark"],  # float64
        "total_width": c["total_width"],
    }


def raw(ref: torch.Tensor, deg: torch.Tensor, c=None):
    """``PesqLoss.raw`` at 16 kHz with the reference's CPU precision mix."""

    c = constants32() if c is None else c
    deg, ref = torch.atleast_2d(deg), torch.atleast_2d(ref)
    max_val = torch.max(deg.abs().amax(1, keepdim=True), ref.abs().amax(1, keepdim=True))
    deg, ref = deg / max_val, ref / max_val

    def align(sig):
        f = _LFilter32.apply(sig, c["power_b"], c["power_a"])
        power = (f**2).sum(dim=1, keepdim=True) / (f.shape[1] + 5120) / 1.04684
        return sig * (10**7 / power).sqrt()

    def preemph(sig):
        emp = torch.linspace(0, 15, 16)[1:] / 16.0
        sig = sig.clone()
        sig[:, :15] = sig[:, :15] * emp
        sig[:, -15:] = sig[:, -15:] * torch.flip(emp, dims=(0,))
        return _LFilter32.apply(sig, c["pre_b"], c["pre_a"])

    ref, deg = preemph(align(ref)), preemph(align(deg))
    ref = torch.nn.functional.pad(ref, (0, ref.shape[1] % 256))
    deg = torch.nn.functional.pad(deg, (0, deg.shape[1] % 256))

    def bark(sig):
        spec = torch.stft(sig, n_fft=512, hop_length=256, win_length=512, window=c["window"],
                          center=False, normalized=False, return_complex=True)
        spec = spec.abs().pow(2).swapaxes(1, 2)
        spec = torch.cat([torch.zeros_like(spec[:, :, :1]), spec[:, :, 1:]], dim=2)
        return torch.matmul(spec[:, :, :-1], c["fbank"].t()) * c["corr"]

    cc = dict(O.constants())
    cc["exp"] = c["exp"]
    return O.chain(bark(ref), bark(deg), cc)


def loss(ref, deg, factor=1.0):
    ds, da = raw(ref, deg)
    return O.epilogue(ds, da, factor)[1]


def mos(ref, deg):
    ds, da = raw(ref, deg)
    return O.epilogue(ds, da, 1.0)[0]
