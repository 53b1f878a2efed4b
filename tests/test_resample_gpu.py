"""GPU parity of the HIP polyphase resampler (the ``TritonResample`` operator).

Oracle: torchaudio's convolution form evaluated in float64 with the same
float32 filter bank (``oracle.pesq_oracle.resample``).  Bound: scale aware,
``|got - want| <= ATOL + RTOL * peak`` with the reference's ``ATOL = 1e-6``,
``RTOL = 2e-6`` (``test_triton_resample.py:36-37``).  Coverage follows
``test_triton_resample.py``: rate pairs with odd lengths, the backward
(adjoint identity), double backward, output lengths, identity at equal rates.
The exact torchaudio taps themselves are parity unpinned (see
``oracle/pesq_oracle.py``).
"""

import ctypes
import math

import numpy as np
import pytest
import torch

from bench import synthetic_config
from oracle import pesq_oracle as O
from torch_pesq import PesqLossTriton
from torch_pesq.hip_ops.resample import HipResample

pytestmark = pytest.mark.gpu

ATOL, RTOL = 1e-6, 2e-6
RATES = [(44100, 16000), (48000, 16000), (8000, 16000), (22050, 16000), (16000, 8000)]


def _close(got, want):
    got = got.double().cpu()
    peak = float(want.abs().max())
    return float((got - want).abs().max()) <= ATOL + RTOL * peak


@pytest.mark.parametrize("orig,new", RATES)
@pytest.mark.parametrize("length", [1, 37, 1001, 44101])
def test_forward_matches_float64(orig, new, length):
    mod = HipResample(orig, new).cuda()
    x = torch.randn(3, length, generator=torch.Generator().manual_seed(length))
    got = mod(x.cuda())
    want = O.resample(x.double(), orig, new)
    assert got.shape == want.shape == (3, O.resample_length(length, orig, new))
    assert _close(got, want)


@pytest.mark.parametrize("orig,new", [(44100, 16000), (22050, 16000), (16000, 44100), (44100, 48000)])
@pytest.mark.parametrize("length", [37, 1001, 44101])
def test_planned_forward_matches_untiled_kernel(orig, new, length):
    """The planned forward (phase major for these many-phase pairs: each phase's
    taps in registers, one output per phase and period) against the untiled
    per-output kernel: both sum the non-zero taps in ascending order in
    float64 (the planned kernel adds exact zeros past a phase's run and for
    samples outside the row), so the outputs are the same numbers."""

    from torch_pesq import _lib

    mod = HipResample(orig, new).cuda()
    x = torch.randn(3, length, generator=torch.Generator().manual_seed(7 * length)).cuda()
    got = mod(x)
    want = torch.empty_like(got)
    lib = _lib.library()
    _lib.check(
        lib.pesq_resample_forward(
            _lib.ptr(x), _lib.ptr(want), 3, length, got.shape[1], _lib.ptr(mod.kernel),
            _lib.ptr(mod.tap_lo), _lib.ptr(mod.tap_hi), mod.orig_step, mod.new_step, mod.width,
            mod.kernel.shape[1], _lib.stream_handle(x.device),
        ),
        "pesq_resample_forward",
    )
    torch.cuda.synchronize()
    assert torch.equal(got, want)


@pytest.mark.parametrize("orig,new", [(44100, 16000), (48000, 16000), (22050, 16000), (8000, 16000)])
@pytest.mark.parametrize("length", [37, 1001, 44101])
def test_pair_calls_match_single_calls(orig, new, length):
    """pesq_resample_plan_forward_pair / _backward_pair (the reference and the
    degraded signal in one launch, as the loss resamples them) against two
    single calls: each row is computed by the same code from its own signal,
    so the outputs are bitwise equal."""

    from torch_pesq import _lib

    mod = HipResample(orig, new).cuda()
    lib = _lib.library()
    gen = torch.Generator().manual_seed(length + orig)
    x0 = torch.randn(3, length, generator=gen).cuda()
    x1 = torch.randn(3, length, generator=gen).cuda()
    n_out = O.resample_length(length, orig, new)
    info = ctypes.byref(mod.plan_info)
    stream = _lib.stream_handle(x0.device)
    pair = [torch.empty(3, n_out, device="cuda") for _ in range(2)]
    single = [torch.empty(3, n_out, device="cuda") for _ in range(2)]
    _lib.check(lib.pesq_resample_plan_forward_pair(
        _lib.ptr(x0), _lib.ptr(pair[0]), _lib.ptr(x1), _lib.ptr(pair[1]), 3, length, n_out, info,
        _lib.ptr(mod.plan), stream), "pesq_resample_plan_forward_pair")
    for x, y in zip((x0, x1), single):
        _lib.check(lib.pesq_resample_plan_forward(
            _lib.ptr(x), _lib.ptr(y), 3, length, n_out, info, _lib.ptr(mod.plan), stream),
            "pesq_resample_plan_forward")
    g0 = torch.randn(3, n_out, generator=gen).cuda()
    g1 = torch.randn(3, n_out, generator=gen).cuda()
    gpair = [torch.empty(3, length, device="cuda") for _ in range(2)]
    gsingle = [torch.empty(3, length, device="cuda") for _ in range(2)]
    _lib.check(lib.pesq_resample_plan_backward_pair(
        _lib.ptr(g0), _lib.ptr(gpair[0]), _lib.ptr(g1), _lib.ptr(gpair[1]), 3, length, n_out,
        info, _lib.ptr(mod.plan), stream), "pesq_resample_plan_backward_pair")
    for g, gx in zip((g0, g1), gsingle):
        _lib.check(lib.pesq_resample_plan_backward(
            _lib.ptr(g), _lib.ptr(gx), 3, length, n_out, info, _lib.ptr(mod.plan), stream),
            "pesq_resample_plan_backward")
    torch.cuda.synchronize()
    for a, b in zip(pair + gpair, single + gsingle):
        assert torch.equal(a, b)
    assert _close(pair[1], O.resample(x1.double().cpu(), orig, new))


@pytest.mark.parametrize("orig", [32000, 48000, 64000, 96000])
@pytest.mark.parametrize("length", [1, 37, 6001, 50001])
def test_integer_decimation(orig, length):
    """Decimation by 2, 3, 4 and 6 to 16 kHz: the single phase plans, whose kernels
    keep a register window of the staged samples (forward) and of the upstream
    gradient (adjoint); lengths below, at and across the workgroup tiles."""

    mod = HipResample(orig, 16000).cuda()
    x = torch.randn(2, length, generator=torch.Generator().manual_seed(orig + length))
    got = mod(x.cuda())
    want = O.resample(x.double(), orig, 16000)
    assert got.shape == want.shape
    assert _close(got, want)
    xg = x.cuda().requires_grad_(True)
    y = mod(xg)
    g = torch.randn(y.shape, generator=torch.Generator().manual_seed(length))
    (gx,) = torch.autograd.grad(y, xg, grad_outputs=g.cuda())
    xo = x.double().requires_grad_(True)
    (gw,) = torch.autograd.grad(O.resample(xo, orig, 16000), xo, grad_outputs=g.double())
    assert _close(gx, gw)


@pytest.mark.parametrize("orig,new", RATES)
def test_backward_is_the_adjoint(orig, new):
    mod = HipResample(orig, new).cuda()
    x = torch.randn(2, 5003, device="cuda", requires_grad=True)
    y = mod(x)
    g = torch.randn_like(y)
    (gx,) = torch.autograd.grad(y, x, grad_outputs=g)
    lhs = float((g.double() * y.double()).sum())
    rhs = float((gx.double() * x.double()).sum())
    assert abs(lhs - rhs) <= 1e-5 * (abs(lhs) + 1.0)
    # against float64 autograd through the oracle's convolution
    xo = x.detach().double().cpu().requires_grad_(True)
    (want,) = torch.autograd.grad(O.resample(xo, orig, new), xo, grad_outputs=g.double().cpu())
    assert _close(gx, want)


def test_double_backward():
    mod = HipResample(44100, 16000).cuda()
    x = torch.randn(1, 3000, device="cuda", requires_grad=True)
    v = torch.randn(1, mod.output_length(3000), device="cuda", requires_grad=True)
    (gx,) = torch.autograd.grad(mod(x), x, grad_outputs=v, create_graph=True)
    u = torch.randn_like(gx)
    (gv,) = torch.autograd.grad(gx, v, grad_outputs=u)
    torch.testing.assert_close(gv, mod(u), rtol=1e-6, atol=1e-7)


def test_identity_and_shapes():
    mod = HipResample(16000, 16000)
    x = torch.randn(2, 100)
    assert mod(x) is x
    m48 = HipResample(48000, 16000).cuda()
    assert m48(torch.zeros(0, 1000, device="cuda")).shape == (0, 334)
    assert m48(torch.randn(2, 3, 1000, device="cuda")).shape == (2, 3, 334)


@pytest.mark.parametrize("orig,new", [(48000, 16000), (44100, 16000), (8000, 16000)])
@pytest.mark.parametrize("shape", [(5001,), (2, 3, 5001), (2, 1, 2, 777)])
def test_leading_dimensions(orig, new, shape):
    """Any number of leading dimensions is packed and unpacked like torchaudio
    (``test_triton_resample.py:556-572``): values and gradients of a
    ``[..., sample]`` input against the float64 oracle on its rows."""

    mod = HipResample(orig, new).cuda()
    x = torch.randn(*shape, generator=torch.Generator().manual_seed(sum(shape)))
    xg = x.cuda().requires_grad_(True)
    y = mod(xg)
    n_out = O.resample_length(shape[-1], orig, new)
    assert y.shape == shape[:-1] + (n_out,)
    rows = x.reshape(-1, shape[-1]).double().requires_grad_(True)
    want = O.resample(rows, orig, new)
    assert _close(y.reshape(-1, n_out), want.detach())
    g = torch.randn(*y.shape, generator=torch.Generator().manual_seed(3))
    (gx,) = torch.autograd.grad(y, xg, grad_outputs=g.cuda())
    (want_g,) = torch.autograd.grad(want, rows, grad_outputs=g.reshape(-1, n_out).double())
    assert gx.shape == shape
    assert _close(gx.reshape(-1, shape[-1]), want_g)


@pytest.mark.parametrize("config,items,samples", [(3, 2, 44100), (5, 3, 48000)])
def test_resampled_pipeline_matches_float64(config, items, samples):
    ref, deg, fs = synthetic_config(config, items=items, samples=samples)
    model = PesqLossTriton(0.5, sample_rate=fs).cuda()
    got = model._run(torch.from_numpy(ref).cuda(), torch.from_numpy(deg).cuda())
    ds, da = O.pipeline(torch.from_numpy(ref), torch.from_numpy(deg), sample_rate=fs)
    mos, loss = O.epilogue(ds, da, 0.5)
    for g, w in zip(got, (ds, da, mos, loss)):
        assert float(((g.double().cpu() - w).abs() / w.abs()).max()) < 1e-5


@pytest.mark.parametrize(
    "orig,new", [(1000, 999), (13, 7), (7, 13), (8000, 11025), (44100, 48000), (2, 1)]
)
def test_exotic_rate_pairs(orig, new):
    """Coprime and near-unity rate pairs (``test_triton_resample.py:650-666``)."""

    mod = HipResample(orig, new).cuda()
    x = torch.randn(2, 3001, generator=torch.Generator().manual_seed(23))
    got = mod(x.cuda())
    want = O.resample(x.double(), orig, new)
    assert got.shape == want.shape
    assert _close(got, want)
    xg = x.cuda().requires_grad_(True)
    y = mod(xg)
    g = torch.randn(y.shape, generator=torch.Generator().manual_seed(orig))
    (gx,) = torch.autograd.grad(y, xg, grad_outputs=g.cuda())
    xo = x.double().requires_grad_(True)
    (gw,) = torch.autograd.grad(O.resample(xo, orig, new), xo, grad_outputs=g.double())
    assert _close(gx, gw)


@pytest.mark.parametrize(
    "options",
    [
        dict(lowpass_filter_width=1),
        dict(lowpass_filter_width=64),
        dict(rolloff=0.5),
        dict(resampling_method="sinc_interp_kaiser", beta=8.0),
        dict(lowpass_filter_width=16, rolloff=0.945, resampling_method="sinc_interp_kaiser"),
    ],
)
@pytest.mark.parametrize("orig,new", [(48000, 16000), (22050, 16000)])
def test_filter_design_variants(orig, new, options):
    """Non default filter designs (``test_triton_resample.py:669-697``); width 64 is the
    longest accumulation (621 taps at 22.05 kHz)."""

    mod = HipResample(orig, new, **options).cuda()
    x = torch.randn(2, 4321, generator=torch.Generator().manual_seed(5))
    got = mod(x.cuda())
    want = O.resample(x.double(), orig, new, **options)
    assert _close(got, want)
    xg = x.cuda().requires_grad_(True)
    y = mod(xg)
    g = torch.randn(y.shape, generator=torch.Generator().manual_seed(7))
    (gx,) = torch.autograd.grad(y, xg, grad_outputs=g.cuda())
    xo = x.double().requires_grad_(True)
    (gw,) = torch.autograd.grad(O.resample(xo, orig, new, **options), xo, grad_outputs=g.double())
    assert _close(gx, gw)


@pytest.mark.parametrize("orig,new", RATES)
def test_output_length_float32_ceil(orig, new):
    """torchaudio's float32 ``ceil`` of the output length, also where it differs
    from the exact integer ceil (above ~180k samples at 44.1 kHz)."""

    mod = HipResample(orig, new).cuda()
    for length in list(range(1, 32)) + [255, 256, 257, 4096, 100_000, 180_000, 180_001,
                                        180_224, 262_144]:
        got = mod(torch.zeros(1, length, device="cuda"))
        assert got.shape == (1, O.resample_length(length, orig, new)), (orig, new, length)


def test_moved_after_construction():
    mod = HipResample(48000, 16000)
    x = torch.randn(2, 4096, device="cuda")
    with pytest.raises(RuntimeError, match="move the module"):
        mod(x)
    mod = mod.cuda()
    assert _close(mod(x), O.resample(x.double().cpu(), 48000, 16000))
