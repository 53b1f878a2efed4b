"""``PesqLossTriton.graphed`` against the eager loss, bit for bit.

Mirrors the reference's graph tests (``tests/test_triton_loss.py:324-337``,
the bit exactness promised at ``triton_ops/loss.py:157-158``): the graphed
callable of one shape and one set of ``requires_grad`` flags gives the eager
loss and gradients exactly, on every replay, with eager work on other inputs
between the replays (which would expose state a replay wrongly keeps), at
16 kHz and through the resampler (48 and 44.1 kHz), for gradients of either
or both inputs and for a forward-only capture.  Also: new data in the inputs
is picked up, both in new tensors (copied into the graph's static inputs) and
in the same buffers passed again (read in place by a graph captured for
them, more buffer pairs than such graphs are kept), non-contiguous and 1-d
inputs, a shape other than the captured one raises, the backward is
differentiable once, and the per stage geometry (``make_graphed_callables``).
``graphed_step`` (forward and backward of ``loss.sum()`` in one graph, not in
the reference) is held to the same: the eager step's bits on every replay,
with new data written into its static inputs.
"""

import pytest
import torch

from bench import speech_like_pair
from torch_pesq import PesqLossTriton

pytestmark = pytest.mark.gpu


def _pair(batch, samples, seed):
    ref, deg = speech_like_pair(batch, samples, seed=seed, noise=0.1)
    return torch.from_numpy(ref).cuda(), torch.from_numpy(deg).cuda()


def _grads(loss, inputs):
    want = [t for t in inputs if t.requires_grad]
    if not want:
        return []
    return list(torch.autograd.grad(loss.sum(), want))


def _check_replays(model, r, d, replays=3):
    eager = model(r, d)
    needs_grad = eager.requires_grad
    eager_grads = [g.clone() for g in _grads(eager, (r, d))]
    eager = eager.detach().clone()
    graphed = model.graphed(r, d)
    for step in range(replays):
        loss = graphed(r, d)
        grads = _grads(loss, (r, d))
        torch.cuda.synchronize()
        assert loss.requires_grad == needs_grad
        assert torch.equal(loss, eager), step
        assert len(grads) == len(eager_grads)
        for want, got in zip(eager_grads, grads):
            assert got.shape == want.shape
            assert torch.equal(got, want), step
        # eager work on other inputs between the replays
        model(r.detach() * 0.5, d.detach() + 0.01)
        torch.cuda.synchronize()
    return graphed


@pytest.mark.parametrize("rate,samples", [(16000, 20000), (48000, 60000), (44100, 55125)])
@pytest.mark.parametrize("flags", [(False, True), (True, True), (True, False), (False, False)])
def test_graphed_matches_eager(rate, samples, flags):
    model = PesqLossTriton(0.5, sample_rate=rate).cuda()
    r, d = _pair(2, samples, seed=31)
    r.requires_grad_(flags[0])
    d.requires_grad_(flags[1])
    _check_replays(model, r, d)


def test_new_input_data_is_picked_up():
    model = PesqLossTriton(0.5, sample_rate=16000).cuda()
    r, d = _pair(3, 16000, seed=32)
    d.requires_grad_(True)
    graphed = model.graphed(r, d)
    for scale in (1.0, 0.5, 2.0):
        d2 = (d.detach() * scale + 0.02 * r).requires_grad_(True)
        want = model(r, d2)
        (want_g,) = torch.autograd.grad(want.sum(), d2)
        got = graphed(r, d2)
        (got_g,) = torch.autograd.grad(got.sum(), d2)
        assert torch.equal(got, want)
        assert torch.equal(got_g, want_g)


def test_same_buffers_with_new_contents():
    """Buffers passed on consecutive calls are read in place; new contents count."""
    model = PesqLossTriton(0.5, sample_rate=48000).cuda()
    r, d = _pair(2, 48000, seed=37)
    buf = d.detach().clone().requires_grad_(True)
    graphed = model.graphed(r, buf)
    for scale in (1.0, 0.5, 2.0, 0.25, 1.5):
        with torch.no_grad():
            buf.copy_(d * scale + 0.02 * r)
        want = model(r, buf)
        (want_g,) = torch.autograd.grad(want.sum(), buf)
        got = graphed(r, buf)
        (got_g,) = torch.autograd.grad(got.sum(), buf)
        assert torch.equal(got, want), scale
        assert torch.equal(got_g, want_g), scale


def test_many_input_buffers():
    """More buffer pairs than graphs kept for them, each used twice in a row."""
    model = PesqLossTriton(0.5, sample_rate=16000).cuda()
    r, d = _pair(2, 16000, seed=38)
    pairs = [(r * (1 + i), (d * (1 + i) + 0.01 * i * r).requires_grad_(True)) for i in range(6)]
    want = []
    for rb, db in pairs:
        loss = model(rb, db)
        (g,) = torch.autograd.grad(loss.sum(), db)
        want.append((loss.detach().clone(), g.clone()))
    graphed = model.graphed(r, pairs[0][1])
    for sweep in range(2):
        for i, (rb, db) in enumerate(pairs):
            for call in range(2):
                loss = graphed(rb, db)
                (g,) = torch.autograd.grad(loss.sum(), db)
                assert torch.equal(loss, want[i][0]), (sweep, i, call)
                assert torch.equal(g, want[i][1]), (sweep, i, call)


def test_noncontiguous_and_1d_inputs():
    model = PesqLossTriton(0.5, sample_rate=16000).cuda()
    r, d = _pair(2, 16010, seed=33)
    rv, dv = r[:, 5:16005], d[:, 3:16003]  # row strided views
    assert not rv.is_contiguous()
    dv = dv.detach().requires_grad_(True)
    eager = model(rv, dv)
    (eager_g,) = torch.autograd.grad(eager.sum(), dv)
    graphed = model.graphed(rv, dv)
    got = graphed(rv, dv)
    (got_g,) = torch.autograd.grad(got.sum(), dv)
    assert torch.equal(got, eager)
    assert torch.equal(got_g, eager_g)

    r1 = r[0].contiguous()
    d1 = d[0].contiguous().requires_grad_(True)
    eager = model(r1, d1)
    (eager_g,) = torch.autograd.grad(eager.sum(), d1)
    graphed = model.graphed(r1, d1)
    got = graphed(r1, d1)
    (got_g,) = torch.autograd.grad(got.sum(), d1)
    assert got.shape == eager.shape == (1,)
    assert got_g.shape == d1.shape
    assert torch.equal(got, eager)
    assert torch.equal(got_g, eager_g)


def test_other_shape_raises():
    model = PesqLossTriton(0.5, sample_rate=16000).cuda()
    r, d = _pair(2, 16000, seed=34)
    graphed = model.graphed(r, d)
    with pytest.raises(RuntimeError, match="shape"):
        graphed(r[:1], d[:1])
    # the module itself still takes any shape
    assert model(r[:1], d[:1]).shape == (1,)


def test_double_backward_raises():
    model = PesqLossTriton(0.5, sample_rate=16000).cuda()
    r, d = _pair(1, 16000, seed=35)
    d.requires_grad_(True)
    graphed = model.graphed(r, d)
    loss = graphed(r, d)
    (plain,) = torch.autograd.grad(loss, d, retain_graph=True)
    plain = plain.clone()
    seed = torch.ones_like(loss).requires_grad_(True)
    (g,) = torch.autograd.grad(loss, d, grad_outputs=seed, create_graph=True)
    assert torch.equal(g.detach(), plain) and g.requires_grad
    with pytest.raises(RuntimeError, match="differentiate twice"):
        g.sum().backward()


def test_per_stage_geometry_graphed():
    model = PesqLossTriton(0.5, sample_rate=16000, n_fft=256, win_length=256, hop_length=128)
    model = model.cuda()
    r, d = _pair(2, 16000, seed=36)
    d.requires_grad_(True)
    _check_replays(model, r, d, replays=2)


@pytest.mark.parametrize("rate,samples", [(16000, 20000), (48000, 60000)])
@pytest.mark.parametrize("flags", [(False, True), (True, True)])
def test_graphed_step_matches_eager(rate, samples, flags):
    """The whole step as one graph: loss and gradients of the eager step, every replay."""
    model = PesqLossTriton(0.5, sample_rate=rate).cuda()
    r, d = _pair(2, samples, seed=39)
    r.requires_grad_(flags[0])
    d.requires_grad_(flags[1])
    step = model.graphed_step(r, d)
    static_r, static_d = step.inputs()
    assert torch.equal(static_r, r.detach()) and torch.equal(static_d, d.detach())
    for scale in (1.0, 1.0, 0.5, 2.0):
        with torch.no_grad():
            static_d.copy_(d * scale + 0.01 * (scale - 1.0) * r)
        rr = static_r.clone().requires_grad_(flags[0])
        dd = static_d.clone().requires_grad_(flags[1])
        want = model(rr, dd)
        want_grads = torch.autograd.grad(want.sum(), [t for t in (rr, dd) if t.requires_grad])
        step.replay()
        torch.cuda.synchronize()
        loss, g_ref, g_deg = step.outputs()
        assert torch.equal(loss, want.detach()), scale
        got_grads = [g for g, f in zip((g_ref, g_deg), flags) if f]
        assert (g_ref is None) == (not flags[0])
        for w, g in zip(want_grads, got_grads):
            assert torch.equal(g, w), scale
        # eager work on other inputs between the replays
        model(r.detach() * 0.5, d.detach() + 0.01)
        torch.cuda.synchronize()


def test_graphed_step_needs_a_gradient():
    model = PesqLossTriton(0.5, sample_rate=16000).cuda()
    r, d = _pair(1, 16000, seed=40)
    with pytest.raises(ValueError, match="gradient"):
        model.graphed_step(r, d)
