"""GPU parity of the stand-alone HIP IIR filter (the ``TritonIIR`` operator).

Oracle: the difference equation in float64 (``scipy.signal.lfilter``, pinned
in ``test_oracle.py``).  Bound: peak relative error ``TOL = 1e-6`` (the
reference's own bound is 1e-5, ``test_triton_iir.py:38-50``); the kernels
keep a float64 state, so what remains is the float32 rounding of the output
(~6e-8).  Coverage follows ``test_triton_iir.py``: both PESQ filters, other
filter families and orders, tile boundary and long lengths, the adjoint,
double backward, strided input, determinism.
"""

import numpy as np
import pytest
import torch
from scipy.signal import butter, cheby1, lfilter

from oracle import pesq_oracle as O
from torch_pesq.hip_ops.iir import HipIIR

pytestmark = pytest.mark.gpu

TOL = 1e-6
C = O.constants()
FILTERS = {
    "power": (C["power_b"].numpy(), C["power_a"].numpy()),
    "pre": (C["pre_b"].numpy(), C["pre_a"].numpy()),
    "lowpass4": butter(4, 0.2),
    "highpass6": butter(6, 0.05, btype="high"),
    "cheby8": cheby1(4, 1.0, [0.1, 0.3], btype="band"),
    "order1": ([0.3, 0.2], [1.0, -0.95]),
    "order16": butter(16, 0.4),
}


def _peak_rel(got, want):
    want = np.asarray(want)
    return float(np.abs(got.double().cpu().numpy() - want).max() / max(np.abs(want).max(), 1e-300))


@pytest.mark.parametrize("name", sorted(FILTERS))
# 1024 samples per scan block: block edges, a partial last block, several blocks
@pytest.mark.parametrize("length", [1, 17, 1023, 1024, 1025, 4097, 20000])
def test_forward_and_adjoint(name, length):
    b, a = FILTERS[name]
    mod = HipIIR(b, a).cuda()
    x = torch.randn(3, length, dtype=torch.float64, generator=torch.Generator().manual_seed(length))
    got = mod(x.float().cuda())
    assert _peak_rel(got, O.lfilter64(x.numpy(), b, a)) < TOL

    xg = x.float().cuda().requires_grad_(True)
    y = mod(xg)
    g = torch.randn(3, length, dtype=torch.float64, generator=torch.Generator().manual_seed(7))
    (gx,) = torch.autograd.grad(y, xg, grad_outputs=g.float().cuda())
    assert _peak_rel(gx, O.lfilter64(g.numpy(), b, a, reverse=True)) < TOL


# up to 128 blocks the output kernel scans the preceding block aggregates
# itself (in groups of 64 blocks); longer rows go through the prefix kernel,
# whose lanes take ceil(blocks / 64) consecutive blocks each: 3 at 132097
# samples (130 blocks: a partial lane, then empty ones), 15 at 960000 (all
# held in registers), 23 at 1.5 M (past the 16 a lane holds)
@pytest.mark.parametrize("length", [65537, 128000, 131072, 132097, 960000, 1_500_000])
def test_long_signals(length):
    b, a = FILTERS["power"]
    mod = HipIIR(b, a).cuda()
    x = np.random.default_rng(1).standard_normal((2, length))
    got = mod(torch.from_numpy(x).float().cuda())
    assert _peak_rel(got, O.lfilter64(x.astype(np.float32), b, a)) < TOL


def test_impulse_step_and_last_sample():
    b, a = FILTERS["power"]
    mod = HipIIR(b, a).cuda()
    n = 9000
    x = np.zeros((3, n), dtype=np.float32)
    x[0, 0] = 1.0          # impulse
    x[1, :] = 1.0          # step
    x[2, n - 1] = 1.0      # last sample only
    got = mod(torch.from_numpy(x).cuda())
    want = lfilter(b, a, x.astype(np.float64), axis=-1)
    assert _peak_rel(got[:2], want[:2]) < TOL
    assert torch.count_nonzero(got[2, : n - 1]) == 0
    assert abs(float(got[2, n - 1]) - b[0] / a[0]) <= 1e-7 * abs(b[0] / a[0])


def test_double_backward_is_the_forward_filter():
    b, a = FILTERS["pre"]
    mod = HipIIR(b, a).cuda()
    x = torch.randn(2, 5000, device="cuda", requires_grad=True)
    v = torch.randn(2, 5000, device="cuda", requires_grad=True)
    y = mod(x)
    (gx,) = torch.autograd.grad(y, x, grad_outputs=v, create_graph=True)
    u = torch.randn(2, 5000, device="cuda")
    (gv,) = torch.autograd.grad(gx, v, grad_outputs=u)
    torch.testing.assert_close(gv, mod(u), rtol=0, atol=0)


def test_strided_and_deterministic():
    b, a = FILTERS["power"]
    mod = HipIIR(b, a).cuda()
    x = torch.randn(4, 20000, device="cuda")
    assert torch.equal(mod(x[:, ::2]), mod(x[:, ::2].contiguous()))
    assert torch.equal(mod(x), mod(x))
    # rows are independent
    assert torch.equal(mod(x)[2:3], mod(x[2:3]))


def test_nan_does_not_cross_rows():
    """A poisoned row does not contaminate its neighbours, forward and adjoint
    (``test_triton_iir.py:574-586``): every scan block belongs to one row."""

    b, a = FILTERS["power"]
    mod = HipIIR(b, a).cuda()
    x = torch.randn(3, 5000, device="cuda")
    x[1, 2500] = float("nan")
    xg = x.clone().requires_grad_(True)
    y = mod(xg)
    assert torch.isfinite(y[0]).all() and torch.isfinite(y[2]).all()
    assert torch.isnan(y[1, 2500:]).any() and torch.isfinite(y[1, :2500]).all()
    g = torch.randn_like(y)
    g[1, 1000] = float("nan")
    (gx,) = torch.autograd.grad(y, xg, grad_outputs=g)
    assert torch.isfinite(gx[0]).all() and torch.isfinite(gx[2]).all()
    # the adjoint runs back in time: the poisoned upstream reaches samples before it
    assert torch.isnan(gx[1, :1001]).any() and torch.isfinite(gx[1, 1001:]).all()


def test_errors():
    mod = HipIIR(*FILTERS["pre"]).cuda()
    with pytest.raises(RuntimeError):
        mod(torch.zeros(2, 100))
    with pytest.raises(RuntimeError):
        mod(torch.zeros(2, 100, device="cuda", dtype=torch.float64))
    with pytest.raises(RuntimeError):
        mod(torch.zeros(2, 3, 100, device="cuda"))
    assert mod(torch.zeros(2, 0, device="cuda")).shape == (2, 0)
