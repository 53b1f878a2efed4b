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


@pytest.mark.parametrize("config,items,samples", [(3, 2, 44100), (5, 3, 48000)])
def test_resampled_pipeline_matches_float64(config, items, samples):
    ref, deg, fs = synthetic_config(config, items=items, samples=samples)
    model = PesqLossTriton(0.5, sample_rate=fs).cuda()
    got = model._run(torch.from_numpy(ref).cuda(), torch.from_numpy(deg).cuda())
    ds, da = O.pipeline(torch.from_numpy(ref), torch.from_numpy(deg), sample_rate=fs)
    mos, loss = O.epilogue(ds, da, 0.5)
    for g, w in zip(got, (ds, da, mos, loss)):
        assert float(((g.double().cpu() - w).abs() / w.abs()).max()) < 1e-5
