"""The loss inside a training loop: a small denoiser trained on SI-SDR + PESQ.

The reference recommends combining the PESQ loss with scale-invariant SDR for
noise suppression (``README.md:11,120-127``).  These tests run that use: a
frame-wise MLP denoiser whose output is scored by ``PesqLossTriton`` next to
an SI-SDR term, gradients flowing from the HIP pipeline into the network's
parameters.

* parameter gradients of one step match the same network evaluated in float64
  on the CPU through the float64 oracle pipeline, at 16 kHz and through the
  48 kHz resampler: ``PARAM_RTOL = 1e-4`` of the largest gradient entry per
  parameter tensor (the network itself runs in float32 on the GPU);
* a step through ``graphed()`` gives bit-identical parameter gradients to the
  eager step, over several steps with optimizer updates and eager work between
  the replays;
* a short Adam run on a fixed batch lowers the combined loss.
"""

import pytest
import torch

from bench import speech_like_pair
from oracle import pesq_oracle as O
from torch_pesq import PesqLossTriton

pytestmark = pytest.mark.gpu

PARAM_RTOL = 1e-4
FACTOR = 1.0
SDR_WEIGHT = 0.01
FRAME = 64


class FrameDenoiser(torch.nn.Module):
    """Residual MLP over non-overlapping frames of ``FRAME`` samples."""

    def __init__(self, hidden: int = 128):
        super().__init__()
        self.inp = torch.nn.Linear(FRAME, hidden)
        self.out = torch.nn.Linear(hidden, FRAME)
        torch.nn.init.normal_(self.out.weight, std=1e-3)
        torch.nn.init.zeros_(self.out.bias)

    def forward(self, noisy: torch.Tensor) -> torch.Tensor:
        frames = noisy.reshape(noisy.shape[0], -1, FRAME)
        return noisy + self.out(torch.tanh(self.inp(frames))).reshape(noisy.shape)


def si_sdr(est: torch.Tensor, ref: torch.Tensor) -> torch.Tensor:
    """Scale-invariant SDR in dB per row (Le Roux et al., arXiv:1811.02508)."""

    alpha = (est * ref).sum(-1, keepdim=True) / (ref * ref).sum(-1, keepdim=True)
    target = alpha * ref
    return 10 * torch.log10((target * target).sum(-1) / ((target - est) ** 2).sum(-1))


def combined(pesq: torch.Tensor, est: torch.Tensor, ref: torch.Tensor) -> torch.Tensor:
    return pesq.mean() - SDR_WEIGHT * si_sdr(est, ref).mean()


def _net(seed: int) -> FrameDenoiser:
    torch.manual_seed(seed)
    return FrameDenoiser()


def _oracle_param_grads(net, ref, noisy, fs):
    """The same step in float64 on the CPU, the loss from the float64 oracle."""

    net64 = FrameDenoiser().double()
    net64.load_state_dict({k: v.detach().double().cpu() for k, v in net.state_dict().items()})
    r = torch.from_numpy(ref).double()
    est = net64(torch.from_numpy(noisy).double())
    ds, da = O.pipeline(r, est, sample_rate=fs)
    _, pesq = O.epilogue(ds, da, FACTOR)
    combined(pesq, est, r).backward()
    return {k: p.grad for k, p in net64.named_parameters()}


@pytest.mark.parametrize("fs,seconds", [(16000, 1.0), (48000, 1.0)])
def test_parameter_gradients_match_float64(fs, seconds):
    samples = int(fs * seconds)
    ref, noisy = speech_like_pair(2, samples, seed=21, noise=0.1, fs=fs)
    net = _net(0).cuda()
    loss_fn = PesqLossTriton(FACTOR, sample_rate=fs).cuda()

    r, x = torch.from_numpy(ref).cuda(), torch.from_numpy(noisy).cuda()
    est = net(x)
    combined(loss_fn(r, est), est, r).backward()
    want = _oracle_param_grads(net, ref, noisy, fs)
    for name, p in net.named_parameters():
        got = p.grad.double().cpu()
        assert torch.isfinite(got).all(), name
        err = float((got - want[name]).abs().max() / want[name].abs().max())
        assert err < PARAM_RTOL, (name, err)


def test_graphed_training_steps_are_bit_exact():
    ref, noisy = speech_like_pair(2, 16000, seed=22, noise=0.1)
    r, x = torch.from_numpy(ref).cuda(), torch.from_numpy(noisy).cuda()
    loss_fn = PesqLossTriton(FACTOR, sample_rate=16000).cuda()

    def run(graphed_loss, steps=3):
        net = _net(1).cuda()
        opt = torch.optim.Adam(net.parameters(), lr=1e-3)
        history = []
        for _ in range(steps):
            opt.zero_grad(set_to_none=True)
            est = net(x)
            pesq = graphed_loss(r, est) if graphed_loss else loss_fn(r, est)
            combined(pesq, est, r).backward()
            history.append([p.grad.clone() for p in net.parameters()] + [pesq.detach().clone()])
            opt.step()
            # eager work between the replays
            loss_fn(r, x)
            torch.cuda.synchronize()
        return history

    eager = run(None)
    sample_est = _net(1).cuda()(x)
    graphed = loss_fn.graphed(r, sample_est)
    for want, got in zip(eager, run(graphed)):
        for w, g in zip(want, got):
            assert torch.equal(g, w)


def test_adam_lowers_combined_loss():
    ref, noisy = speech_like_pair(4, 16000, seed=23, noise=0.2)
    r, x = torch.from_numpy(ref).cuda(), torch.from_numpy(noisy).cuda()
    loss_fn = PesqLossTriton(FACTOR, sample_rate=16000).cuda()
    net = _net(2).cuda()
    opt = torch.optim.Adam(net.parameters(), lr=2e-3)
    values = []
    for _ in range(30):
        opt.zero_grad(set_to_none=True)
        est = net(x)
        loss = combined(loss_fn(r, est), est, r)
        loss.backward()
        values.append(float(loss))
        opt.step()
    assert all(torch.isfinite(torch.tensor(values)))
    assert values[-1] < values[0], values
    mos = loss_fn.mos(r, net(x).detach())
    assert ((mos > 1) & (mos < 5)).all()
