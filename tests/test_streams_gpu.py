"""The loss on PyTorch's current stream, whichever it is.

The reference enqueues all work on the current stream and keeps no state
between calls that two streams could share (``iir.py:945-963``,
``triton_ops/loss.py:182-199``).  Checked here: the loss
and its gradients computed under a side stream equal the default stream's
bit for bit (the backward runs on the forward's stream), two streams working
on different batches at the same time each get their own results (the
workspaces are per call, nothing is shared), through the resampler too, and
the graphed loss replays on a side stream.
"""

import pytest
import torch

from bench import speech_like_pair
from torch_pesq import PesqLossTriton

pytestmark = pytest.mark.gpu


def _pair(batch, samples, seed, noise=0.1):
    ref, deg = speech_like_pair(batch, samples, seed=seed, noise=noise)
    return torch.from_numpy(ref).cuda(), torch.from_numpy(deg).cuda()


def _step(model, r, d):
    d = d.detach().requires_grad_(True)
    loss = model(r, d)
    (g,) = torch.autograd.grad(loss.sum(), d)
    return loss.detach(), g


@pytest.mark.parametrize("rate,samples", [(16000, 24000), (48000, 72000)])
def test_side_stream_matches_default(rate, samples):
    model = PesqLossTriton(0.5, sample_rate=rate).cuda()
    r, d = _pair(3, samples, seed=41)
    want_loss, want_g = _step(model, r, d)
    torch.cuda.synchronize()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        loss, g = _step(model, r, d)
    side.synchronize()
    assert torch.equal(loss, want_loss)
    assert torch.equal(g, want_g)


@pytest.mark.parametrize("rate,samples", [(16000, 32000), (48000, 96000)])
def test_two_streams_at_once(rate, samples):
    model = PesqLossTriton(0.5, sample_rate=rate).cuda()
    batches = [_pair(4, samples, seed=42 + i, noise=0.05 + 0.1 * i) for i in range(2)]
    want = [_step(model, r, d) for r, d in batches]
    torch.cuda.synchronize()
    streams = [torch.cuda.Stream() for _ in batches]
    for s in streams:
        s.wait_stream(torch.cuda.current_stream())
    got = [None, None]
    # interleave the two streams' launches, no synchronisation between them
    for rep in range(3):
        for i, ((r, d), s) in enumerate(zip(batches, streams)):
            with torch.cuda.stream(s):
                got[i] = _step(model, r, d)
    torch.cuda.synchronize()
    for (want_loss, want_g), (loss, g) in zip(want, got):
        assert torch.equal(loss, want_loss)
        assert torch.equal(g, want_g)
    assert not torch.equal(want[0][0], want[1][0])


def test_graphed_on_a_side_stream():
    model = PesqLossTriton(0.5, sample_rate=16000).cuda()
    r, d = _pair(2, 20000, seed=44)
    want_loss, want_g = _step(model, r, d)
    d = d.detach().requires_grad_(True)
    graphed = model.graphed(r, d)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for _ in range(3):
            loss = graphed(r, d)
            (g,) = torch.autograd.grad(loss.sum(), d)
            loss, g = loss.clone(), g.clone()
    side.synchronize()
    assert torch.equal(loss, want_loss)
    assert torch.equal(g, want_g)
